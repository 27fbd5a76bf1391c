"""Llama-3 scaled RoPE table and interleaved rotation (test infrastructure only).

Restates ``rope_cache`` (app/engine.py:28-43) with its precision sequence:

    freqs = 1.0 / (base ** (arange(0, hd, 2)[:hd//2].float() / hd))   # fp32 tensor ops
    per frequency f (Python float): wl = 2*pi/f
        wl < old/high -> f;  wl > old/low -> f/scale;
        else s = (old/wl - low)/(high - low), (1 - s)*f/scale + s*f
    theta = fp32(...);  idx = fp32(pos) * theta (fp32);  table = stack([cos, sin], -1)

pow, cos and sin are evaluated in float64 and rounded once to float32.  ``apply_rope``
restates app/engine.py:46-53 (pairs (x[2i], x[2i+1]) rotated in fp32, cast back).
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import f16


def rope_freqs(head_dim: int, base=500_000, scale=32, low=1, high=4, old=8192) -> np.ndarray:
    """The scaled inverse frequencies theta [head_dim // 2] (float32)."""
    e = np.arange(0, head_dim, 2)[: head_dim // 2].astype(np.float32) / np.float32(head_dim)
    p = np.power(np.float64(np.float32(base)), e.astype(np.float64)).astype(np.float32)
    freqs = (np.float32(1.0) / p).astype(np.float32)
    lo_w, hi_w = old / low, old / high
    out = []
    for f in freqs.tolist():
        wl = 2 * math.pi / f
        if wl < hi_w:
            out.append(f)
        elif wl > lo_w:
            out.append(f / scale)
        else:
            s = (old / wl - low) / (high - low)
            out.append((1 - s) * f / scale + s * f)
    return np.asarray(out, dtype=np.float32)


def rope_cache(head_dim: int, max_seq: int, **kw) -> np.ndarray:
    """Table [max_seq, head_dim // 2, 2] float32 of (cos, sin)."""
    theta = rope_freqs(head_dim, **kw)
    idx = (np.arange(max_seq, dtype=np.float32)[:, None] * theta[None, :]).astype(np.float32)
    ang = idx.astype(np.float64)
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def apply_rope(x, cs) -> np.ndarray:
    """x [..., HD] fp16, cs [..., HD/2, 2] (broadcastable) -> fp16 rotated pairs."""
    xs = np.asarray(x, dtype=np.float32).reshape(*np.shape(x)[:-1], -1, 2)
    c, s = cs[..., 0], cs[..., 1]
    o0 = xs[..., 0] * c - xs[..., 1] * s
    o1 = xs[..., 1] * c + xs[..., 0] * s
    return f16(np.stack([o0, o1], -1).reshape(np.shape(x)))
