"""The reference's CPU path restated in numpy float32 (test infrastructure only).

HeartMuLaLite on ``device="cpu"`` (app/engine.py:215-265 with fast = False) dequantises
every int8 layer once at load, ``w = (q8.float() * s8.float()[:, None]).to(dtype)``
(:242), and runs ``F.linear`` (:72), torch ``rms`` (:56-58), ``apply_rope`` (:46-53) and
SDPA over the cache (:136-149).  This module restates that computation in float32
(numpy has no bfloat16; the reference picks bf16 on CPU, :222) for two uses:

* a second oracle with the slow-path semantics, to cross-check the fast-path oracle
  (``oracle.model``) -- they must agree within fp16-level noise;
* the CPU baseline timed next to the GPU numbers (the reference's own CPU path, bounded
  to a sample of layers and scaled to a frame).
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import bf16_to_f32
from .rope import rope_cache


def dequant(q8, s_bits) -> np.ndarray:
    """app/engine.py:242: q8.float() * s8.float()[:, None] (here kept in float32)."""
    return (np.asarray(q8, np.float32) * bf16_to_f32(s_bits)[:, None]).astype(np.float32)


def rms(x, w, eps=1e-5):
    """app/engine.py:56-58 in float32."""
    x = np.asarray(x, np.float32)
    return (x / np.sqrt((x * x).mean(-1, keepdims=True) + np.float32(eps))).astype(np.float32) * w


def apply_rope(x, cs):
    xs = x.reshape(*x.shape[:-1], -1, 2)
    c, s = cs[..., 0], cs[..., 1]
    return np.stack([xs[..., 0] * c - xs[..., 1] * s, xs[..., 1] * c + xs[..., 0] * s],
                    -1).reshape(x.shape).astype(np.float32)


class CpuBlock:
    def __init__(self, w, pre, heads, kv_heads, dim):
        def lin(n):
            return dequant(w[pre + n + ".q8"], w[pre + n + ".s8"])
        self.wqkv = np.concatenate([lin(f"attn.{n}_proj.weight") for n in ("q", "k", "v")])
        self.wo = lin("attn.output_proj.weight")
        self.w13 = np.concatenate([lin("mlp.w1.weight"), lin("mlp.w3.weight")])
        self.w2 = lin("mlp.w2.weight")
        self.n1 = bf16_to_f32(w[pre + "sa_norm.scale"])
        self.n2 = bf16_to_f32(w[pre + "mlp_norm.scale"])
        self.h, self.kvh, self.hd = heads, kv_heads, dim // heads
        self.kc = self.vc = None

    def alloc(self, B, L):
        self.kc = np.zeros((B, self.kvh, L, self.hd), np.float32)
        self.vc = np.zeros_like(self.kc)

    def __call__(self, x, pos, rope):
        """One step for x [B, D] at per-row positions pos [B] (S = 1 decode, app/engine.py:123-153
        with the GQA-without-copy branch :138-142)."""
        B = x.shape[0]
        Hq, Hk, HD = self.h, self.kvh, self.hd
        h = rms(x, self.n1)
        qkv = h @ self.wqkv.T
        cs = rope[pos][:, None]
        q = apply_rope(qkv[:, : Hq * HD].reshape(B, Hq, HD), cs)
        k = apply_rope(qkv[:, Hq * HD:(Hq + Hk) * HD].reshape(B, Hk, HD), cs)
        v = qkv[:, (Hq + Hk) * HD:].reshape(B, Hk, HD)
        G = Hq // Hk
        o = np.empty((B, Hq, HD), np.float32)
        for b in range(B):
            p = int(pos[b])
            self.kc[b, :, p] = k[b]
            self.vc[b, :, p] = v[b]
            kk = self.kc[b, :, : p + 1]                                # [Hk, T, HD]
            vv = self.vc[b, :, : p + 1]
            qg = q[b].reshape(Hk, G, HD)
            sc = np.einsum("hgd,htd->hgt", qg, kk) / np.float32(math.sqrt(HD))
            sc = np.exp(sc - sc.max(-1, keepdims=True))
            sc /= sc.sum(-1, keepdims=True)
            o[b] = np.einsum("hgt,htd->hgd", sc, vv).reshape(Hq, HD)
        x = x + o.reshape(B, Hq * HD) @ self.wo.T
        a = rms(x, self.n2) @ self.w13.T
        F = a.shape[1] // 2
        av = a[:, :F]
        return x + ((av / (1 + np.exp(-av))) * a[:, F:]) @ self.w2.T


class CpuStack:
    def __init__(self, w, prefix, cfg, layers=None):
        n = cfg["layers"] if layers is None else layers
        self.blocks = [CpuBlock(w, f"{prefix}.layers.{i}.", cfg["heads"], cfg["kv_heads"], cfg["dim"])
                       for i in range(n)]
        self.norm = bf16_to_f32(w[f"{prefix}.norm.scale"])
        self.hd = cfg["dim"] // cfg["heads"]
        self.rope = None

    def alloc(self, B, L):
        self.rope = rope_cache(self.hd, max(L, 16))
        for b in self.blocks:
            b.alloc(B, L)

    def decode(self, x, pos):
        x = np.asarray(x, np.float32)
        for b in self.blocks:
            x = b(x, np.asarray(pos), self.rope)
        return rms(x, self.norm)
