"""Write tests/golden/decode_vectors.npz: small seeded input/output vectors of every oracle
function on the decode path (the reference ships no tests or golden vectors, so these are
produced by the pinned oracle and guard it -- and the GPU kernels -- against drift).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import kernels as K  # noqa: E402
from oracle.model import cfg_mix, sample  # noqa: E402
from oracle.quant import q8_rows, scale_f16  # noqa: E402
from oracle.rope import rope_cache  # noqa: E402

OUT = Path(__file__).resolve().parent / "decode_vectors.npz"


def vectors() -> dict:
    g = np.random.default_rng(2024)
    v = {}
    # quantiser: a row with exact ties, a zero row, random rows
    s = 2.0 ** -7
    w = (g.standard_normal((6, 128)) * 0.02).astype(np.float32)
    w[0, :8] = np.array([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5], np.float32) * s
    w[0, 8:] = 0
    w[1] = 0
    v["q8_w"] = w
    v["q8_q"], v["q8_s"] = q8_rows(w)
    # GEMV, both numerics, with residual
    q, sb = q8_rows((g.standard_normal((96, 256)) * 0.02).astype(np.float32))
    sc = scale_f16(sb)
    v["gemv_q"], v["gemv_s"] = q, sc
    for M in (8, 20):
        x = g.standard_normal((M, 256)).astype(np.float16)
        r = g.standard_normal((M, 96)).astype(np.float16)
        v[f"gemv_x{M}"], v[f"gemv_r{M}"] = x, r
        v[f"gemv_y{M}"] = K.gemv_i8(x, q, sc, r)
    # RMSNorm
    x = (g.standard_normal((4, 512)) * 2).astype(np.float16)
    nw = (1 + 0.05 * g.standard_normal(512)).astype(np.float16)
    v["rms_x"], v["rms_w"], v["rms_y"] = x, nw, K.rms(x, nw)
    # RoPE table and cache write
    v["rope_tab"] = rope_cache(128, 40)
    qkv = g.standard_normal((4, (4 + 2 * 2) * 128)).astype(np.float16)
    kc = g.standard_normal((2, 2, 40, 128)).astype(np.float16)
    vc = g.standard_normal((2, 2, 40, 128)).astype(np.float16)
    pos = np.array([5, 6, 30, 31], np.int64)
    v["rope_qkv"], v["rope_pos"], v["rope_kc0"], v["rope_vc0"] = qkv, pos, kc.copy(), vc.copy()
    v["rope_q"] = K.rope_kv_write(qkv, v["rope_tab"], pos, kc, vc, 2, 4, 2, 128)
    v["rope_kc"], v["rope_vc"] = kc, vc
    # decode attention (GQA 3:1, 16 splits) over the written caches
    qa = g.standard_normal((2, 6 * 128)).astype(np.float16)
    ka = g.standard_normal((2, 2, 300, 128)).astype(np.float16)
    va = g.standard_normal((2, 2, 300, 128)).astype(np.float16)
    pa = np.array([299, 117], np.int64)
    v["attn_q"], v["attn_k"], v["attn_v"], v["attn_pos"] = qa, ka, va, pa
    v["attn_o"] = K.decode_attn_out(qa, ka, va, pa, 1, 6, 2, 128, nsplit=16)
    # SiLU * mul
    xs = (g.standard_normal((3, 2 * 200)) * 3).astype(np.float16)
    v["silu_x"], v["silu_y"] = xs, K.silu_mul(xs)
    # sampler with injected noise, CFG 1.5, top-50
    lg = (g.standard_normal((4, 8197)) * 3).astype(np.float16)
    nz = g.exponential(1.0, (2, 8197)).astype(np.float32)
    v["smp_logits"], v["smp_noise"] = lg, nz
    v["smp_tok"] = sample(cfg_mix(lg, 2, 1.5).astype(np.float32), 50, 1.0, nz)
    return v


if __name__ == "__main__":
    np.savez_compressed(OUT, **vectors())
    print(f"wrote {OUT} ({OUT.stat().st_size / 1024:.0f} KB)")
