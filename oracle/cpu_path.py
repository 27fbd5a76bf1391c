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


# ---------------------------------------------------------------- slow-path frame (fast = False)
def _forward_block(blk, x, pos, rope, attn_len, mask):
    """Block.__call__ (app/engine.py:123-153) in float32: x [B, S, D], pos [B, S] absolute
    positions (the cache write uses pos[0] for the whole batch, :133-135), attention over the
    first attn_len cache slots with ``mask`` [B, 1, S, attn_len] (True = attend) or, with
    mask None, SDPA's top-left causal mask (:148).  Both SDPA branches (:138-149) give query
    head h the kv head h // G, so one repeat-based form covers them."""
    B, S, _ = x.shape
    Hq, Hk, HD = blk.h, blk.kvh, blk.hd
    G = Hq // Hk
    h = rms(x, blk.n1)
    qkv = h @ blk.wqkv.T
    cs = rope[pos][:, :, None]                                        # [B, S, 1, HD/2, 2]
    q = apply_rope(qkv[..., : Hq * HD].reshape(B, S, Hq, HD), cs)
    k = apply_rope(qkv[..., Hq * HD:(Hq + Hk) * HD].reshape(B, S, Hk, HD), cs)
    v = qkv[..., (Hq + Hk) * HD:].reshape(B, S, Hk, HD)
    p0 = np.asarray(pos[0])
    blk.kc[:, :, p0] = k.transpose(0, 2, 1, 3)
    blk.vc[:, :, p0] = v.transpose(0, 2, 1, 3)
    kk = np.repeat(blk.kc[:, :, :attn_len], G, axis=1)                # [B, Hq, T, HD]
    vv = np.repeat(blk.vc[:, :, :attn_len], G, axis=1)
    sc = q.transpose(0, 2, 1, 3) @ kk.transpose(0, 1, 3, 2) / np.float32(math.sqrt(HD))
    if mask is None:
        allow = np.tril(np.ones((S, attn_len), bool))[None, None]
    else:
        allow = np.asarray(mask, bool)
    sc = np.where(allow, sc, -np.inf).astype(np.float32)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = (p @ vv).transpose(0, 2, 1, 3).reshape(B, S, Hq * HD)
    x = x + o @ blk.wo.T
    a = rms(x, blk.n2) @ blk.w13.T
    F = a.shape[-1] // 2
    av = a[..., :F]
    return (x + ((av / (1 + np.exp(-av))) * a[..., F:]) @ blk.w2.T).astype(np.float32)


def stack_forward(stack, x, pos, attn_len, mask):
    """Stack.__call__ (app/engine.py:174-178): rc = rope[pos], every block, final rms."""
    x = np.asarray(x, np.float32)
    for b in stack.blocks:
        x = _forward_block(b, x, np.asarray(pos, np.int64), stack.rope, attn_len, mask)
    return rms(x, stack.norm)


class CpuModel:
    """HeartMuLaLite's slow path (``fast = False``) in float32, under teacher forcing:

        _step          app/engine.py:350-354  codebook sum, masked backbone call (S = 1)
        _frame_from_h  app/engine.py:311-326  c0 head; the depth decoder called as
                                              Stack.__call__ on the growing sequence with
                                              dec_mask (:265, :320-321); audio_head[i - 1]
                                              on the last row; positions advance by one

    It shares nothing with the fast-path oracle (``oracle.model``) but the weights, so the
    two pin each other's frame composition: which hidden state feeds which pass, which head
    reads it and at which decoder position."""

    N_CB = 8
    VOCAB = 8197

    def __init__(self, w, backbone_cfg, decoder_cfg):
        self.backbone = CpuStack(w, "backbone", backbone_cfg)
        self.decoder = CpuStack(w, "decoder", decoder_cfg)
        self.projection = dequant(w["projection.weight.q8"], w["projection.weight.s8"])
        self.c0_head = dequant(w["codebook0_head.weight.q8"], w["codebook0_head.weight.s8"])
        self.audio_head = [dequant(w[f"audio_head.{i}.q8"], w[f"audio_head.{i}.s8"])
                           for i in range(self.N_CB - 1)]
        # Emb (app/engine.py:98): q8 rows times their scale
        self.emb_q8 = np.asarray(w["audio_embeddings.weight.q8"])
        self.emb_s = bf16_to_f32(w["audio_embeddings.weight.s8"])
        self.dec_mask = np.tril(np.ones((self.N_CB, self.N_CB), bool))   # :265
        self.B = self.L = None

    def alloc(self, B, L):
        self.B, self.L = B, L
        self.backbone.alloc(B, L)
        self.decoder.alloc(B, self.N_CB)

    def embed_audio(self, cb, tok):
        """_embed_audio (app/engine.py:307-308): rows tok + cb * 8197 -> [B, S, D]."""
        r = np.asarray(tok, np.int64) + cb * self.VOCAB
        return self.emb_q8[r].astype(np.float32) * self.emb_s[r][..., None]

    def frame_from_h(self, last_h, forced):
        """app/engine.py:311-326 with the samples replaced by ``forced`` [B, 8]; returns the
        8 logit sets [B, V] (float32)."""
        B = self.B
        forced = np.asarray(forced, np.int64)
        logits = [last_h @ self.c0_head.T]
        cur = np.concatenate([last_h[:, None], self.embed_audio(0, forced[:, :1])], 1)
        pos = np.broadcast_to(np.arange(2), (B, 2))
        for i in range(1, self.N_CB):
            S = cur.shape[1]
            mask = np.broadcast_to(self.dec_mask[pos[0]][None, None, :, : self.N_CB],
                                   (B, 1, S, self.N_CB))
            h = stack_forward(self.decoder, cur @ self.projection.T, pos, self.N_CB, mask)
            logits.append(h[:, -1] @ self.audio_head[i - 1].T)
            cur = self.embed_audio(i, forced[:, i:i + 1])
            pos = pos[:, -1:] + 1
        return logits

    def step(self, tok, pos, forced):
        """_step (app/engine.py:350-354): tok [B, 8] previous frame at scalar position pos."""
        B = self.B
        rows = np.asarray(tok, np.int64) + np.arange(self.N_CB)[None] * self.VOCAB
        h = (self.emb_q8[rows].astype(np.float32) * self.emb_s[rows][..., None]).sum(1)[:, None]
        mask = (np.arange(self.L)[None, :] <= pos)[None, None].repeat(B, 0)   # [B, 1, 1, L]
        hb = stack_forward(self.backbone, h, np.full((B, 1), pos, np.int64), self.L, mask)
        return self.frame_from_h(hb[:, -1], forced)
