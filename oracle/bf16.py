"""bf16 emulation in numpy (test infrastructure only; see oracle/__init__.py).

torch rounds every bf16 tensor op's fp32 result to bf16 with round-to-nearest-even; the
reference's bf16 blend / scale expressions (llm/src/lastkv/llm/modeling.py:96, :117-119) are
sequences of such ops.  Pinned by: tests/test_oracle_cpu.py compares ``round_bf16`` with torch's
own ``tensor.to(torch.bfloat16)`` on random, tie, overflow and NaN inputs.
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as the float32 value of that bf16."""

    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def to_bits(x) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float32 values."""

    x = np.asarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def from_bits(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def mul(a, b) -> np.ndarray:
    """torch bf16 ``a * b``: fp32 product, one rounding."""

    return round_bf16(np.asarray(a, np.float32) * np.asarray(b, np.float32))


def add(a, b) -> np.ndarray:
    """torch bf16 ``a + b``: fp32 sum, one rounding."""

    return round_bf16(np.asarray(a, np.float32) + np.asarray(b, np.float32))


def rsub(a, scalar: float = 1.0) -> np.ndarray:
    """torch bf16 ``scalar - a``."""

    return round_bf16(np.float32(scalar) - np.asarray(a, np.float32))
