"""Pins for the oracle's quantiser (app/convert_final.py:17-21) and RoPE table / rotation
(app/engine.py:28-53).  Each check comes from the mathematics, not from the oracle's code:
exact ties, closed-form values, invariants and hand-built cases that a plausible slip fails."""
import math

import numpy as np
import pytest

from oracle.numerics import bf16_bits, bf16_to_f32, f16
from oracle.quant import fp32_scale, q8_rows, scale_f16
from oracle.rope import apply_rope, rope_cache, rope_freqs


# ---------------------------------------------------------------- q8_rows
def test_q8_exact_ties_round_half_to_even():
    # amax = 127 * 2^-7 -> s = 2^-7 exactly; w = (k + 1/2) * 2^-7 divides to an exact tie
    s = 2.0 ** -7
    row = np.array([127 * s, 2.5 * s, 3.5 * s, -2.5 * s, -3.5 * s, 0.5 * s, -0.5 * s, 126.5 * s],
                   np.float32)
    q, sb = q8_rows(row[None])
    assert q[0].tolist() == [127, 2, 4, -2, -4, 0, 0, 126]      # half away from zero: 3, 4, -3, ...
    assert bf16_to_f32(sb)[0] == np.float32(s)


def test_q8_clamp_and_zero_row():
    q, sb = q8_rows(np.zeros((1, 9), np.float32))
    assert (q == 0).all()
    assert bf16_to_f32(sb)[0] == bf16_to_f32(bf16_bits(np.array([1e-8], np.float32) / np.float32(127)))[0]
    w = np.random.default_rng(0).standard_normal((64, 300), dtype=np.float32)
    q, _ = q8_rows(w)
    assert np.abs(q.astype(int)).max() == 127
    assert (np.abs(q.astype(int)).max(1) == 127).all()          # the row max maps to +-127
    qn, sbn = q8_rows(-w)
    assert np.array_equal(qn, -q)                                # sign symmetry
    assert np.array_equal(sbn, q8_rows(w)[1])


def test_q8_codes_use_the_unrounded_fp32_scale():
    """The codes divide by the fp32 scale; only the stored scale is rounded to bf16."""
    w = np.random.default_rng(1).standard_normal((256, 512), dtype=np.float32) * np.float32(0.02)
    q, sb = q8_rows(w)
    s32 = (np.abs(w).max(1) / np.float32(127)).astype(np.float32)
    assert np.array_equal(q, np.clip(np.rint(w / s32[:, None]), -127, 127).astype(np.int8))
    alt = np.clip(np.rint(w / bf16_to_f32(sb)[:, None]), -127, 127).astype(np.int8)
    assert (alt != q).any()                                      # a bf16-scale divide would differ
    err = np.abs(q.astype(np.float64) * s32[:, None] - w)
    assert (err <= s32[:, None] * 0.5 * (1 + 1e-6)).all()        # |w - q s| <= s / 2


def test_bf16_round_to_nearest_even():
    bits = np.array([0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001], np.uint32).view(np.float32)
    assert bf16_bits(bits).tolist() == [0x3F80, 0x3F82, 0x3F80, 0x3F81]   # truncation: 3F80, 3F81, ...
    assert scale_f16(np.array([0x3C00], np.uint16))[0] == np.float16(2.0 ** -7)


# ---------------------------------------------------------------- RoPE
def test_rope_frequency_bands_closed_form():
    hd = 128
    th = rope_freqs(hd).astype(np.float64)
    f = np.array([1.0 / (500000.0 ** (2 * i / hd)) for i in range(hd // 2)])
    wl = 2 * math.pi / f
    assert th[0] == 1.0                                          # highest frequency untouched
    hi = wl < 8192 / 4
    lo = wl > 8192 / 1
    np.testing.assert_allclose(th[hi], f[hi], rtol=1e-6)         # wl < old/high: unchanged
    np.testing.assert_allclose(th[lo], f[lo] / 32, rtol=1e-6)    # wl > old/low: divided by scale
    mid = ~hi & ~lo
    assert mid.any()
    # the smoothing band interpolates between f/scale and f: strictly inside, monotone in i
    assert (th[mid] < f[mid] * (1 + 1e-6)).all() and (th[mid] > f[mid] / 32 * (1 - 1e-6)).all()
    assert (np.diff(th) <= 0).all()


def test_rope_table_layout_and_identities():
    t = rope_cache(128, 64).astype(np.float64)
    assert t.shape == (64, 64, 2)
    assert np.array_equal(t[0, :, 0], np.ones(64)) and np.array_equal(t[0, :, 1], np.zeros(64))
    np.testing.assert_allclose(t[..., 0] ** 2 + t[..., 1] ** 2, 1.0, atol=1e-6)
    th = rope_freqs(128).astype(np.float64)
    np.testing.assert_allclose(t[5, :, 0], np.cos(5 * th), atol=2e-6)    # cos first, sin second
    np.testing.assert_allclose(t[5, :, 1], np.sin(5 * th), atol=2e-6)
    # angle additivity: rot(p + q) = rot(p) rot(q)
    c = t[3, :, 0] * t[4, :, 0] - t[3, :, 1] * t[4, :, 1]
    s = t[3, :, 1] * t[4, :, 0] + t[3, :, 0] * t[4, :, 1]
    np.testing.assert_allclose(c, t[7, :, 0], atol=1e-5)
    np.testing.assert_allclose(s, t[7, :, 1], atol=1e-5)


def test_apply_rope_rotates_interleaved_pairs():
    cs = np.zeros((4, 2), np.float32)
    cs[:, 0] = [1, 0, -1, math.cos(0.3)]
    cs[:, 1] = [0, 1, 0, math.sin(0.3)]
    x = np.array([1, 2, 1, 0, 3, -1, 0.5, 0.25], np.float16)    # pairs (x[2i], x[2i+1])
    y = apply_rope(x, cs).astype(np.float64)
    assert y[:2].tolist() == [1, 2]                              # angle 0
    assert y[2:4].tolist() == [0, 1]                             # (1, 0) by 90 degrees -> (0, 1)
    assert y[4:6].tolist() == [-3, 1]                            # 180 degrees
    want = [0.5 * math.cos(0.3) - 0.25 * math.sin(0.3), 0.25 * math.cos(0.3) + 0.5 * math.sin(0.3)]
    np.testing.assert_allclose(y[6:], want, atol=1e-3)
    xs = np.random.default_rng(2).standard_normal((3, 128)).astype(np.float16)
    ys = apply_rope(xs, rope_cache(128, 40)[37][None]).astype(np.float64)
    n_in = (xs.astype(np.float64).reshape(3, 64, 2) ** 2).sum(-1)
    n_out = (ys.reshape(3, 64, 2) ** 2).sum(-1)
    np.testing.assert_allclose(n_out, n_in, rtol=4e-3, atol=1e-3)   # pair norms preserved
