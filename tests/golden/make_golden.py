"""Writes the golden fixtures under tests/golden/ from the reference tests' own closed forms.

The reference (zacharydenton/krea2-hrx) stores no vectors for the W8A8 path; its
tests compute their expectations from closed forms on generated inputs. This script
restates those tests' generators and expectations in numpy (f64 / binary16
arithmetic, independent of the oracle in oracle/) and saves inputs + expected
outputs as compressed .npz files:

  plain_kat_{2048,6144,16384}.npz  tests/quantized.rs:514-569 (bit-exact codes and scale)
  kronecker_{norm,gated,plain}.npz tests/quantized.rs:385-512 (f64 rotated rows, scales)
  gemm_{plain,resid,swiglu}_*.npz  tests/quantized.rs:171-280 (int32 dots, f64 expectations)
  convrot_kat_{6144,16384}.npz     src/training/quantized.rs:124-224 (exact base projection)

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)


def values(n: int, scale: float) -> np.ndarray:
    """tests/quantized.rs:80-82, in f32: ((i*37 % 101) - 50) * scale / 50."""
    i = np.arange(n, dtype=np.int64)
    v = (i * 37 % 101).astype(np.float32) - np.float32(50.0)
    return (v * np.float32(scale)) / np.float32(50.0)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round f64 (or f32) values directly to the nearest bf16 (8 significant bits), ties to even."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)
    return np.ldexp(np.rint(m * 256.0) / 256.0, e)


def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """bf16::from_f32 (round to nearest even on the f32 bit pattern), as uint16 bits."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def plain_kat(width: int) -> dict:
    """tests/quantized.rs:521-567."""
    tokens, stride = 3, width + 64
    i = np.arange(tokens * width, dtype=np.int64)
    scale = np.array([0.0, 0.5, 0.00001], dtype=np.float32)[i // width]
    x32 = (((i * 37 % 101).astype(np.float32) - np.float32(50.0)) * scale) / np.float32(50.0)
    inp = x32.astype(np.float16)
    codes = np.zeros((tokens, width), np.int8)
    scales = np.zeros(tokens, np.float32)
    for t in range(tokens):
        row = inp[t * width:(t + 1) * width].copy()
        for step in (1, 4, 16, 64):
            blocks = row.reshape(-1, 4, step).astype(np.float64)  # [block][j][col]
            out = np.empty_like(blocks)
            for r in range(4):
                s = np.zeros_like(blocks[:, 0, :])
                for j in range(4):
                    s = s + H4[r, j] * blocks[:, j, :]
                out[:, r, :] = s * 0.25
            row = out.astype(np.float16).reshape(-1)  # f64 -> f16, round to nearest even
        mx = np.max(np.abs(row.astype(np.float32)))
        s = np.float32(max(np.float32(mx * np.float32(16.0)), np.float32(1e-30))) / np.float32(127.0)
        inv = np.float32(16.0) / np.float32(s)
        codes[t] = np.clip(np.rint(row.astype(np.float32) * inv), -127, 127).astype(np.int8)
        scales[t] = s
    return dict(width=width, stride=stride, tokens=tokens, h=inp.view(np.uint16), codes=codes,
                scales=scales)


def coefficient_matrix() -> np.ndarray:
    """tests/quantized.rs:391-399: the 256x256 Kronecker-H4 matrix divided by 16."""
    c = np.ones((256, 256))
    ii, jj = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    a, b = ii.copy(), jj.copy()
    for _ in range(4):
        c *= H4[a % 4, b % 4]
        a //= 4
        b //= 4
    return c / 16.0


def kronecker() -> dict:
    """tests/quantized.rs:385-512: inputs, f64 rotated rows and f64 scales per kind."""
    tokens, width, stride = 3, 2048, 2176
    norm_input = bf16_bits_from_f32(values(tokens * width, 1.5))
    half_input = values(tokens * width, 0.5).astype(np.float16)
    norm = values(width, 0.1)
    modulation = values(width, 0.2)
    shift = values(width, 0.15)
    gate = values(tokens * stride, 0.7).astype(np.float16)
    gate_stride = stride + 128
    padded = np.zeros(tokens * gate_stride, np.float16)
    for t in range(tokens):
        padded[t * gate_stride:t * gate_stride + width] = gate[t * stride:t * stride + width]
    coeff = coefficient_matrix()
    out = {}
    for kind in ("norm", "gated", "plain"):
        formed = np.zeros((tokens, width))
        for t in range(tokens):
            x = bf16_from_bits(norm_input[t * width:(t + 1) * width]).astype(np.float64)
            ms = np.sum(x * x) / width
            if kind == "norm":
                normalized = round_bf16(x / np.sqrt(ms + 1e-5) * (1.0 + norm.astype(np.float64)))
                formed[t] = round_bf16(round_bf16(round_bf16(1.0 + modulation.astype(np.float64))
                                                  * normalized) + shift.astype(np.float64))
            elif kind == "gated":
                att = round_bf16(half_input[t * width:(t + 1) * width].astype(np.float64))
                g = gate[t * stride:t * stride + width].astype(np.float64)
                sig = round_bf16(1.0 / (1.0 + np.exp(-g)))
                formed[t] = round_bf16(att * sig)
            else:
                formed[t] = half_input[t * width:(t + 1) * width].astype(np.float64)
        rotated = np.einsum("tgj,ij->tgi", formed.reshape(tokens, width // 256, 256), coeff)
        rotated = rotated.reshape(tokens, width)
        scale = np.maximum(np.max(np.abs(rotated), axis=1), 1e-30) / 127.0
        out[kind] = dict(tokens=tokens, width=width, stride=stride, gate_stride=gate_stride,
                         norm_input=norm_input, half_input=half_input.view(np.uint16), norm=norm,
                         modulation=modulation, shift=shift, gate=padded.view(np.uint16),
                         rotated=rotated, scale=scale)
    return out


def gemm_cases():
    """tests/quantized.rs:175-259: integer operands, dots and expected outputs."""
    cases = []
    for mode, wide in (("plain", False), ("resid", False), ("swiglu", False), ("resid", True)):
        for m, k, n, pad in ((17, 128, 128, 0), (257, 384, 256, 128)):
            n = n * 2 if wide else n
            stride = k + pad
            a = ((np.arange(m * stride) * 3 % 15) - 7).astype(np.int8)
            w = ((np.arange(n * stride) * 7 % 15) - 7).astype(np.int8)
            ws = np.full(n, 0.01, np.float32)
            ws[3] = 0.0
            sc = np.full(m, 0.02, np.float32)
            sc[m - 1] = 0.0
            residual = bf16_bits_from_f32(values(m * n, 0.5))
            gates = values(n, 0.3)
            dot = (a.reshape(m, stride)[:, :k].astype(np.int64)
                   @ w.reshape(n, stride)[:, :k].astype(np.int64).T)
            full = dot.astype(np.float64) * ws.astype(np.float64)[None, :] * sc.astype(np.float64)[:, None]
            if mode == "resid":
                lin = bf16_from_bits(bf16_bits_from_f32(full.astype(np.float32)))
                gated = bf16_from_bits(bf16_bits_from_f32((gates[None, :] * lin).astype(np.float32)))
                tot = bf16_from_bits(residual).reshape(m, n) + gated
                want = bf16_from_bits(bf16_bits_from_f32(tot.astype(np.float32))).astype(np.float64)
            elif mode == "swiglu":
                half = n // 2
                c = np.arange(half)
                gc = (c // 16) * 32 + c % 16
                ga = round_bf16(full[:, gc])
                ub = round_bf16(full[:, gc + 16])
                want = round_bf16(round_bf16(ga / (1.0 + np.exp(-ga))) * ub)
            else:
                want = round_bf16(full)
            name = f"gemm_{mode}{'_wide' if wide else ''}_{m}x{k}x{n}_pad{pad}"
            cases.append((name, dict(m=m, k=k, n=n, stride=stride, a=a, w=w, ws=ws, a_scale=sc,
                                     residual=residual, gates=gates, dot=dot.astype(np.int32),
                                     want=want.astype(np.float32))))
    return cases


def convrot_kat(inputs: int) -> dict:
    """src/training/quantized.rs:131-222, the base (W8A8) projection only."""
    tokens, outputs = 3, 128
    weights = ((np.arange(outputs * inputs) * 37 % 31) - 15).astype(np.int8)
    scales = ((np.arange(outputs) % 7 + 1) / 256.0).astype(np.float32)
    i = np.arange(tokens * inputs)
    x32 = np.where(i < inputs, np.float32(0.0),
                   ((i * 17 % 97).astype(np.float32) - np.float32(48.0)) / np.float32(128.0))
    x = bf16_bits_from_f32(x32.astype(np.float32))
    h = bf16_from_bits(x).astype(np.float16)  # lora_transport: bf16 -> f16
    base = np.zeros((tokens, outputs), np.uint16)
    wm = weights.reshape(outputs, inputs).astype(np.int64)
    for t in range(tokens):
        rotated = h[t * inputs:(t + 1) * inputs].copy()
        for step in (1, 4, 16, 64):
            blocks = rotated.reshape(-1, 4, step).astype(np.float64)
            out = np.empty_like(blocks)
            for r in range(4):
                s = np.zeros_like(blocks[:, 0, :])
                for j in range(4):
                    s = s + H4[r, j] * blocks[:, j, :]
                out[:, r, :] = s * 0.25
            rotated = out.astype(np.float16).reshape(-1)
        mx = np.max(np.abs(rotated.astype(np.float32)))
        scale = np.float32(max(np.float32(mx * np.float32(16.0)), np.float32(1e-30))) / np.float32(127.0)
        codes = np.clip(np.rint(rotated.astype(np.float32) * (np.float32(16.0) / scale)), -127, 127)
        dot = wm @ codes.astype(np.int64)
        base[t] = bf16_bits_from_f32((dot.astype(np.float32) * scales) * scale)
    return dict(inputs=inputs, tokens=tokens, outputs=outputs, weights=weights, scales=scales,
                x_bf16=x, h=h.view(np.uint16), base_bf16=base)


def main() -> None:
    for width in (2048, 6144, 16384):
        np.savez_compressed(os.path.join(HERE, f"plain_kat_{width}.npz"), **plain_kat(width))
    for kind, d in kronecker().items():
        np.savez_compressed(os.path.join(HERE, f"kronecker_{kind}.npz"), **d)
    for name, d in gemm_cases():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **d)
    for inputs in (6144, 16384):
        np.savez_compressed(os.path.join(HERE, f"convrot_kat_{inputs}.npz"), **convrot_kat(inputs))


if __name__ == "__main__":
    main()
