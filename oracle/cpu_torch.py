"""The reference's CPU path on torch (test infrastructure; bench.py times it as the CPU baseline).

HeartMuLaLite on ``device="cpu"`` takes ``fast = False`` (app/engine.py:224-228): every int8
layer is dequantised once at load, ``(q8.float() * s8.float()[:, None]).to(dtype)`` (:242), in
the CPU dtype (bf16 by default, :222), and a frame is

* the backbone step of ``_step`` (:350-354): the 8 codebook rows summed in the model dtype, one
  position, SDPA over the cache with a position mask;
* ``_frame_from_h`` (:311-326): the c0 head, then the depth decoder called as
  ``Stack.__call__`` on the growing sequence with ``dec_mask`` (:265, :320-321), each codebook
  read by ``audio_head[i - 1]`` on the last row, sampled by ``_guided`` / ``_sample``
  (:291-305);
* each block as ``Block.__call__`` (:123-153): torch rms (:56-58), interleaved RoPE
  (:46-53), the cache written at ``pos[0]`` (:133-135), SDPA with the query heads of a kv head
  as a sequence when S == 1 and with repeated kv heads otherwise (:136-149).

It is restated here on torch CPU ops (``F.linear``, ``F.scaled_dot_product_attention``) so the
CPU arithmetic timed beside the GPU is the reference's own, in bf16 or fp16.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .rope import rope_cache

VOCAB = 8197
N_CB = 8


def _deq(w, name, dt):
    """:242 -- int8 codes times the per-row scale, in the model dtype."""
    return (w[name + ".q8"].float() * w[name + ".s8"].float()[:, None]).to(dt)


def _rms(x, g, eps=1e-5):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * g


def _rotate(x, cs):
    """x [B, S, H, D], cs [B, S, D/2, 2]: interleaved pairs rotated in fp32, cast back."""
    p = x.float().unflatten(-1, (-1, 2))
    c, s = cs[..., 0].unsqueeze(2), cs[..., 1].unsqueeze(2)
    return torch.stack((p[..., 0] * c - p[..., 1] * s, p[..., 1] * c + p[..., 0] * s),
                       -1).flatten(-2).to(x.dtype)


class _Layer:
    def __init__(self, w, pre, cfg, dt):
        self.H, self.Hk = cfg["heads"], cfg["kv_heads"]
        self.hd = cfg["dim"] // cfg["heads"]
        self.wqkv = torch.cat([_deq(w, pre + f"attn.{n}_proj.weight", dt) for n in "qkv"])
        self.wo = _deq(w, pre + "attn.output_proj.weight", dt)
        self.w13 = torch.cat([_deq(w, pre + "mlp.w1.weight", dt), _deq(w, pre + "mlp.w3.weight", dt)])
        self.w2 = _deq(w, pre + "mlp.w2.weight", dt)
        self.g1 = w[pre + "sa_norm.scale"].to(dt)
        self.g2 = w[pre + "mlp_norm.scale"].to(dt)
        self.kc = self.vc = None

    def alloc(self, B, L, dt):
        self.kc = torch.zeros(B, self.Hk, L, self.hd, dtype=dt)
        self.vc = torch.zeros_like(self.kc)

    def __call__(self, x, pos, cs, span, mask):
        B, S, _ = x.shape
        H, Hk, hd = self.H, self.Hk, self.hd
        q, k, v = F.linear(_rms(x, self.g1), self.wqkv).split([H * hd, Hk * hd, Hk * hd], -1)
        q = _rotate(q.reshape(B, S, H, hd), cs)
        k = _rotate(k.reshape(B, S, Hk, hd), cs)
        slots = pos[0]
        self.kc[:, :, slots] = k.transpose(1, 2)
        self.vc[:, :, slots] = v.reshape(B, S, Hk, hd).transpose(1, 2)
        kk, vv = self.kc[:, :, :span], self.vc[:, :, :span]
        G = H // Hk
        if S == 1 and G > 1:
            o = F.scaled_dot_product_attention(q.reshape(B, Hk, G, hd), kk, vv, attn_mask=mask)
            o = o.reshape(B, 1, H * hd)
        else:
            o = F.scaled_dot_product_attention(
                q.transpose(1, 2), kk.repeat_interleave(G, 1), vv.repeat_interleave(G, 1),
                attn_mask=mask, is_causal=mask is None and S > 1)
            o = o.transpose(1, 2).reshape(B, S, H * hd)
        x = x + F.linear(o, self.wo)
        a, b = F.linear(_rms(x, self.g2), self.w13).chunk(2, -1)
        return x + F.linear(F.silu(a) * b, self.w2)


class _Stack:
    def __init__(self, w, prefix, cfg, dt):
        self.layers = [_Layer(w, f"{prefix}.layers.{i}.", cfg, dt) for i in range(cfg["layers"])]
        self.g = w[f"{prefix}.norm.scale"].to(dt)
        self.hd = cfg["dim"] // cfg["heads"]
        self.table = None

    def alloc(self, B, L, dt):
        self.table = torch.from_numpy(rope_cache(self.hd, max(L, 16)))
        for layer in self.layers:
            layer.alloc(B, L, dt)

    def __call__(self, x, pos, span, mask):
        cs = self.table[pos]
        for layer in self.layers:
            x = layer(x, pos, cs, span, mask)
        return _rms(x, self.g)


class CpuTorchModel:
    """The reference's CPU frame on torch in ``dtype`` (bf16 is the reference's CPU default).
    ``w`` holds CPU tensors in the int8 file layout (``.q8`` int8, ``.s8`` / norms bf16)."""

    def __init__(self, w, backbone_cfg, decoder_cfg, dtype=torch.bfloat16):
        self.dt = dtype
        self.backbone = _Stack(w, "backbone", backbone_cfg, dtype)
        self.decoder = _Stack(w, "decoder", decoder_cfg, dtype)
        self.projection = _deq(w, "projection.weight", dtype)
        self.c0_head = _deq(w, "codebook0_head.weight", dtype)
        self.audio_head = [_deq(w, f"audio_head.{i}", dtype) for i in range(N_CB - 1)]
        self.eq8 = w["audio_embeddings.weight.q8"]
        self.es = w["audio_embeddings.weight.s8"].to(dtype)
        self.dec_mask = torch.tril(torch.ones(N_CB, N_CB, dtype=torch.bool))
        self.N = self.B = self.L = None

    def alloc(self, n, L, cfg_scale=1.5):
        self.N = n
        self.B = 2 * n if cfg_scale != 1.0 else n
        self.L = L
        self.backbone.alloc(self.B, L, self.dt)
        self.decoder.alloc(self.B, N_CB, self.dt)

    def _emb(self, rows):
        """Emb (:98): int8 rows in the model dtype times their scale."""
        return F.embedding(rows, self.eq8).to(self.dt) * F.embedding(rows, self.es[:, None])

    def _pick(self, logits, cfg, topk, temp, gen):
        """_guided / _sample (:291-305): CFG mix of the cond/uncond rows in the model dtype, then
        top-k, softmax of log_softmax and the exponential race; the token goes to both rows."""
        N = self.N
        if self.B == 2 * N:
            logits = logits[N:] + (logits[:N] - logits[N:]) * cfg
        lg = logits.float() / temp
        cut = torch.topk(lg, topk)[0][..., -1:]
        lg = lg.masked_fill(lg < cut, -math.inf)
        p = torch.softmax(torch.log_softmax(lg, -1), -1)
        e = torch.empty_like(p).exponential_(1, generator=gen)
        t = torch.argmax(p / e, -1, keepdim=True)
        return torch.cat([t, t]) if self.B == 2 * N else t

    @torch.inference_mode()
    def step(self, tok, pos, cfg=1.5, topk=50, temp=1.0, gen=None, forced=None, logits=None):
        """One frame (:345-354 with fast = False): tok [B, 8] of the previous frame at scalar
        position pos -> the frame's tokens [B, 8].  ``forced`` [B, 8] replaces the samples
        (teacher forcing); ``logits`` (a list) collects the 8 logit sets."""
        B = self.B

        def pick(i, lg):
            if logits is not None:
                logits.append(lg)
            if forced is not None:
                return forced[:, i:i + 1]
            return self._pick(lg, cfg, topk, temp, gen)

        rows = tok + torch.arange(N_CB) * VOCAB
        h = self._emb(rows).sum(1, dtype=self.dt).unsqueeze(1)
        mask = (torch.arange(self.L) <= pos)[None, None, None].expand(B, 1, 1, self.L)
        last = self.backbone(h, torch.full((B, 1), pos), self.L, mask)[:, -1]
        out = [pick(0, F.linear(last, self.c0_head))]
        cur = torch.stack([last, self._emb(out[0][:, 0])], 1)
        p = torch.arange(2).expand(B, 2)
        for i in range(1, N_CB):
            S = cur.shape[1]
            m = self.dec_mask[p[0]][None, None].expand(B, 1, S, N_CB)
            hd = self.decoder(F.linear(cur, self.projection), p, N_CB, m)
            out.append(pick(i, F.linear(hd[:, -1], self.audio_head[i - 1])))
            cur = self._emb(out[-1] + i * VOCAB)
            p = p[:, -1:] + 1
        return torch.cat(out, 1)
