"""The transformer launch-shape rules (``src/kernels/shape.rs``), from the library.

Each function calls the C ABI so the Python host, the C++ host and the kernels
share one implementation of the rules.
"""

from __future__ import annotations

from ._lib import lib


def gemm_pitch(k: int) -> int:
    """Operand row pitch in int8 elements (``shape.rs:105-107``)."""
    return int(lib().k2w8_shape_gemm_pitch(k))


def capacity(tokens: int) -> int:
    """Buffer rows for a sequence (``shape.rs:12-16``)."""
    return int(lib().k2w8_shape_capacity(tokens))


def gemm_grid_rows(tokens: int) -> int:
    """Launch grid rows for ``tokens`` rows of activations (``shape.rs:110-112``)."""
    return int(lib().k2w8_shape_gemm_grid_rows(tokens))


def gemm_schedule_rows(tokens: int) -> bool:
    """Whether the wide down projection runs its scheduled variant (``shape.rs:97-99``)."""
    return bool(lib().k2w8_shape_gemm_schedule_rows(tokens))


def gemm_rows() -> int:
    """``GEMM_ROWS`` (``shape.rs:36``)."""
    return int(lib().k2w8_shape_gemm_rows())


def gemm_m_group() -> int:
    """``GEMM_M_GROUP`` (``shape.rs:93``)."""
    return int(lib().k2w8_shape_gemm_m_group())


def tokens_range() -> range:
    """``TOKENS`` (``shape.rs:8``), inclusive bounds as a Python range."""
    lo, hi = int(lib().k2w8_shape_tokens_min()), int(lib().k2w8_shape_tokens_max())
    return range(lo, hi + 1)
