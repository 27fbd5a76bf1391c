"""Per-row symmetric int8 quantiser (test infrastructure only).

Restates ``q8_rows`` of app/convert_final.py:17-21:

    tf = t.float()
    s  = tf.abs().amax(1).clamp(min=1e-8) / 127        # fp32
    q  = (tf / s[:, None]).round().clamp(-127, 127)     # fp32 divide, round half to even
    return q.to(int8), s.to(bfloat16)

and the loader cast of the scales to fp16 (app/engine.py:241, ``s8.to(dtype)``).
The codes use the unrounded fp32 scale; only the stored scale is rounded to bf16.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16_bits, bf16_to_f32, f16


def q8_rows(w) -> tuple[np.ndarray, np.ndarray]:
    """w [N, K] -> (q int8 [N, K], s bf16 bits uint16 [N])."""
    tf = np.asarray(w, dtype=np.float32)
    if tf.ndim != 2:
        raise ValueError("q8_rows expects a 2-D tensor")
    amax = np.abs(tf).max(axis=1) if tf.shape[1] else np.zeros(tf.shape[0], np.float32)
    s = np.maximum(amax, np.float32(1e-8)).astype(np.float32) / np.float32(127)
    q = np.rint(tf / s[:, None].astype(np.float32))
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, bf16_bits(s)


def scale_f16(s_bits) -> np.ndarray:
    """bf16 scale bits -> fp16 as the loader does (``s8.to(torch.float16)``)."""
    return f16(bf16_to_f32(s_bits))


def fp32_scale(w) -> np.ndarray:
    """The unrounded fp32 per-row scale the codes are computed with."""
    tf = np.asarray(w, dtype=np.float32)
    return np.maximum(np.abs(tf).max(axis=1), np.float32(1e-8)).astype(np.float32) / np.float32(127)
