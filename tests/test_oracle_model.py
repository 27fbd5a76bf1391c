"""Pins for the frame-level oracle (app/engine.py): two independent restatements must agree
(fast-path numerics vs the reference's CPU path), structural equivalences the reference's
semantics imply (prompt pass == token-by-token decode; the two-row first decoder pass == two
sequential single-row passes) and the sampler's closed-form special cases."""
import numpy as np
import pytest

from helpers import model_weights_np, tiny_cfgs
from oracle.cpu_path import CpuStack
from oracle.model import OModel, cfg_mix, sample

V = 8197


@pytest.fixture(scope="module")
def tiny():
    bb, dec = tiny_cfgs()
    return bb, dec, model_weights_np(bb, dec, seed=11)


def test_fast_path_agrees_with_cpu_path(tiny):
    bb, dec, w = tiny
    om = OModel(w, bb, dec)
    om.alloc(2, 24)
    cs = CpuStack(w, "backbone", bb)
    cs.alloc(4, 24)
    g = np.random.default_rng(0)
    for p in range(5):                                   # several positions: caches must agree too
        x = g.standard_normal((4, bb["dim"])).astype(np.float16)
        fast = om.backbone.decode(x, np.full(4, p, np.int64), 1).astype(np.float32)
        slow = cs.decode(x.astype(np.float32), np.full(4, p))
        np.testing.assert_allclose(fast, slow, atol=3e-2, rtol=3e-2)


def test_prompt_pass_equals_token_by_token_decode(tiny):
    bb, dec, w = tiny
    a = OModel(w, bb, dec)
    a.alloc(1, 32)
    b = OModel(w, bb, dec)
    b.alloc(1, 32)
    P = 9
    x = np.random.default_rng(1).standard_normal((2, P, bb["dim"])).astype(np.float16)
    pre = a.backbone.prefill(x, np.arange(P, dtype=np.int64)).astype(np.float32)
    for t in range(P):
        step = b.backbone.decode(x[:, t], np.full(2, t, np.int64), 1).astype(np.float32)
        np.testing.assert_allclose(step, pre[:, t], atol=2e-2, rtol=2e-2)
    for la, lb in zip(a.backbone.blocks, b.backbone.blocks):
        np.testing.assert_allclose(la.kc[:, :, :P].astype(np.float32), lb.kc[:, :, :P].astype(np.float32),
                                   atol=2e-2, rtol=2e-2)


def test_first_decoder_pass_two_rows_equal_two_sequential_passes(tiny):
    """decode(x, pos=[0,1]*B, S=2) attends row 2b+1 over slots {0, 1} of batch b; it must equal
    running position 0 then position 1 one row per batch entry (app/engine.py:336-337)."""
    bb, dec, w = tiny
    a = OModel(w, bb, dec)
    a.alloc(2, 24)
    b = OModel(w, bb, dec)
    b.alloc(2, 24)
    B = a.B
    x = np.random.default_rng(2).standard_normal((2 * B, dec["dim"])).astype(np.float16)
    two = a.decoder.decode(x, np.tile(np.arange(2, dtype=np.int64), B), 2)
    s0 = b.decoder.decode(x[0::2], np.zeros(B, np.int64), 1)
    s1 = b.decoder.decode(x[1::2], np.ones(B, np.int64), 1)
    assert np.array_equal(two[0::2], s0)
    assert np.array_equal(two[1::2], s1)


def test_sampler_special_cases():
    g = np.random.default_rng(3)
    lg = (g.standard_normal((2, V)) * 3).astype(np.float32)
    ones = np.ones((2, V), np.float32)
    assert np.array_equal(sample(lg, 50, 1.0, ones)[:, 0], lg.argmax(-1))      # no noise: greedy
    assert np.array_equal(sample(lg, 1, 1.0, g.exponential(1.0, (2, V)))[:, 0], lg.argmax(-1))
    c = (g.standard_normal((3, V)) * 2).astype(np.float16)
    u = (g.standard_normal((3, V)) * 2).astype(np.float16)
    both = np.concatenate([c, u])
    assert np.array_equal(cfg_mix(both, 3, 0.0), u)                             # cfg 0 -> uncond
    mixed = cfg_mix(both, 3, 1.5).astype(np.float64)
    np.testing.assert_allclose(mixed, u + 1.5 * (c.astype(np.float64) - u), atol=2e-2, rtol=2e-3)
    # never outside the top-k set
    for _ in range(20):
        t = sample(lg, 5, 0.8, g.exponential(1.0, (2, V)))[:, 0]
        for r in range(2):
            assert lg[r, t[r]] >= np.sort(lg[r])[-5]


def test_sampler_distribution_monte_carlo():
    g = np.random.default_rng(4)
    row = (g.standard_normal(V) * 1.5).astype(np.float32)
    n = 4000
    draws = sample(np.tile(row, (n, 1)), 20, 1.3, g.exponential(1.0, (n, V)).astype(np.float32))[:, 0]
    top = np.argsort(-row)[:20]
    p = np.exp((row[top] - row[top].max()) / 1.3)
    p /= p.sum()
    freq = np.array([(draws == t).mean() for t in top])
    assert np.isin(draws, top).all()
    assert 0.5 * np.abs(freq - p).sum() < 0.04
