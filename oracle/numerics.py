"""Rounding helpers shared by the oracle (test infrastructure only).

numpy's float16 conversion rounds to nearest even, and any fp16 op evaluated in float32
then rounded once to fp16 equals the correctly rounded fp16 op (float32 has at least
2*11+2 significand bits), so ``f16(a op b)`` below reproduces native fp16 arithmetic.
"""
from __future__ import annotations

import numpy as np


def f16(a) -> np.ndarray:
    """Round to IEEE binary16, nearest even."""
    return np.asarray(a, dtype=np.float32).astype(np.float16)


def f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit pattern (uint16), round to nearest even (finite inputs),
    as torch's ``.to(torch.bfloat16)``."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def hmul(a, b) -> np.ndarray:
    """fp16 x fp16 -> fp16 (single rounding)."""
    return f16(f32(a) * f32(b))


def hadd(a, b) -> np.ndarray:
    return f16(f32(a) + f32(b))


def hsub(a, b) -> np.ndarray:
    return f16(f32(a) - f32(b))
