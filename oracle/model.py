"""Frame-level oracle: static-cache Llama stacks, sampling and the per-frame step
(test infrastructure only).

Restates app/engine.py:
    Linear / fuse / Emb            :62-104   (int8 codes + per-row fp16 scales)
    Block / Stack (prefill)        :108-178  (SDPA semantics: exact causal softmax attention)
    Stack.decode                   :180-211  (the fast path the HIP kernels implement)
    _sample / _guided              :291-305
    _embed_audio / _frame_fast     :307-343
    _step                          :345-349
on weights held as a dict in the reference's file format (``<name>.q8`` int8,
``<name>.s8`` bf16 bits as uint16, norm scales as bf16 bits, app/convert_final.py:32-47).
"""
from __future__ import annotations

import math

import numpy as np

from . import kernels as K
from .numerics import bf16_to_f32, f16, f32, hadd, hmul, hsub
from .quant import scale_f16
from .rope import rope_cache

AUDIO_VOCAB = 8197
N_CB = 8


class OLinear:
    def __init__(self, q, s16):
        self.q, self.s = np.asarray(q, np.int8), np.asarray(s16, np.float16)

    def __call__(self, x, res=None):
        return K.gemv_i8(x, self.q, self.s, res)


def fuse(parts):
    """app/engine.py:82-86: row concatenation (q|k|v, w1|w3)."""
    return OLinear(np.concatenate([p.q for p in parts]), np.concatenate([p.s for p in parts]))


class OBlock:
    def __init__(self, p, pre, heads, kv_heads, dim):
        self.qkv = fuse([p(pre + f"attn.{n}_proj.weight") for n in ("q", "k", "v")])
        self.o = p(pre + "attn.output_proj.weight")
        self.w13 = fuse([p(pre + "mlp.w1.weight"), p(pre + "mlp.w3.weight")])
        self.w2 = p(pre + "mlp.w2.weight")
        self.n1 = p(pre + "sa_norm.scale", norm=True)
        self.n2 = p(pre + "mlp_norm.scale", norm=True)
        self.h, self.kvh, self.hd = heads, kv_heads, dim // heads
        self.kc = self.vc = None

    def alloc(self, B, L):
        self.kc = np.zeros((B, self.kvh, L, self.hd), np.float16)
        self.vc = np.zeros_like(self.kc)


class OStack:
    def __init__(self, p, prefix, cfg):
        dim = cfg["dim"]
        self.blocks = [OBlock(p, f"{prefix}.layers.{i}.", cfg["heads"], cfg["kv_heads"], dim)
                       for i in range(cfg["layers"])]
        self.norm = p(f"{prefix}.norm.scale", norm=True)
        self.hd = dim // cfg["heads"]
        self.nsplit = 16 if cfg["max_seq"] > 64 else 1
        self.rope = None

    def alloc(self, B, L):
        self.rope = rope_cache(self.hd, max(L, 16))
        for b in self.blocks:
            b.alloc(B, L)

    def decode(self, x, pos, S, nsplit=None):
        """Stack.decode (app/engine.py:180-211): x [R, D] fp16, row r -> batch r // S."""
        ns = self.nsplit if nsplit is None else nsplit
        x = np.asarray(x, np.float16)
        pos = np.asarray(pos, np.int64)
        for b in self.blocks:
            Hq, Hk, HD = b.h, b.kvh, b.hd
            qkv = b.qkv(K.rms(x, b.n1))
            q = K.rope_kv_write(qkv, self.rope, pos, b.kc, b.vc, S, Hq, Hk, HD)
            o = K.decode_attn_out(q, b.kc, b.vc, pos, S, Hq, Hk, HD, nsplit=ns)
            x = b.o(o, res=x)
            a = b.w13(K.rms(x, b.n2))
            x = b.w2(K.silu_mul(a), res=x)
        return K.rms(x, self.norm)

    def prefill(self, x, pos):
        """Stack.__call__ with mask=None (app/engine.py:123-153, :174-178): causal prompt pass,
        x [B, P, D] fp16, pos [P] shared by the batch; attention is the exact softmax
        (SDPA semantics), written to the cache like index_copy_ (:133-135)."""
        x = np.asarray(x, np.float16)
        B, P, D = x.shape
        pos = np.asarray(pos, np.int64)
        cs = self.rope[pos]                                            # [P, HD/2, 2]
        from .rope import apply_rope
        for b in self.blocks:
            Hq, Hk, HD = b.h, b.kvh, b.hd
            h = K.rms(x.reshape(B * P, D), b.n1)
            qkv = b.qkv(h).reshape(B, P, -1)
            q = apply_rope(qkv[..., : Hq * HD].reshape(B, P, Hq, HD), cs[None, :, None])
            k = apply_rope(qkv[..., Hq * HD:(Hq + Hk) * HD].reshape(B, P, Hk, HD), cs[None, :, None])
            v = qkv[..., (Hq + Hk) * HD:].reshape(B, P, Hk, HD)
            b.kc[:, :, pos] = k.transpose(0, 2, 1, 3)
            b.vc[:, :, pos] = v.transpose(0, 2, 1, 3)
            G = Hq // Hk
            o = np.zeros((B, P, Hq, HD), np.float64)
            for bb in range(B):
                for hh in range(Hq):
                    kk = b.kc[bb, hh // G, : pos[-1] + 1].astype(np.float64)
                    vv = b.vc[bb, hh // G, : pos[-1] + 1].astype(np.float64)
                    qq = q[bb, :, hh].astype(np.float64)
                    sc = qq @ kk.T / math.sqrt(HD)
                    sc = np.where(np.arange(kk.shape[0])[None, :] <= pos[:, None], sc, -np.inf)
                    pr = np.exp(sc - sc.max(1, keepdims=True))
                    o[bb, :, hh] = (pr @ vv) / pr.sum(1, keepdims=True)
            o = f16(o.astype(np.float32)).reshape(B * P, Hq * HD)
            xf = b.o(o, res=x.reshape(B * P, D))
            a = b.w13(K.rms(xf, b.n2))
            x = b.w2(K.silu_mul(a), res=xf).reshape(B, P, D)
        return K.rms(x.reshape(B * P, D), self.norm).reshape(B, P, D)


def sample(logits, topk, temp, noise):
    """_sample (app/engine.py:291-298) with the Exponential(1) draws supplied as `noise`:
    argmax(softmax(log_softmax(masked logits / temp)) / noise)."""
    lg = f32(logits) / np.float32(temp)
    thr = np.sort(lg, axis=-1)[..., -topk][..., None]
    lg = np.where(lg < thr, np.float32(-np.inf), lg).astype(np.float32)
    mx = lg.max(-1, keepdims=True)
    ls = (lg - mx - np.log(np.exp(lg - mx).sum(-1, keepdims=True))).astype(np.float32)
    e = np.exp(ls - ls.max(-1, keepdims=True))
    probs = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    return np.argmax(probs / f32(noise), -1)[..., None].astype(np.int64)


def cfg_mix(logits, N, cfg):
    """The CFG mix of _guided (app/engine.py:303) in fp16: u + (c - u) * cfg."""
    lg = np.asarray(logits, np.float16)
    c, u = lg[:N], lg[N:]
    return hadd(u, f16(f32(hsub(c, u)) * np.float32(cfg)))


class OModel:
    """HeartMuLaLite's fast path on numpy (app/engine.py:215-349)."""

    def __init__(self, weights: dict, backbone_cfg: dict, decoder_cfg: dict):
        self.w = weights

        def p(name, norm=False):
            if norm:
                return f16(bf16_to_f32(weights[name]))
            return OLinear(weights[name + ".q8"], scale_f16(weights[name + ".s8"]))

        self.backbone = OStack(p, "backbone", backbone_cfg)
        self.decoder = OStack(p, "decoder", decoder_cfg)
        if "audio_embeddings.weight" in weights:     # dense table (--keep-emb-bf16 files)
            self.audio_dense = f16(bf16_to_f32(weights["audio_embeddings.weight"]))
            self.audio_q8 = self.audio_s = None
        else:
            self.audio_dense = None
            self.audio_q8 = weights["audio_embeddings.weight.q8"]
            self.audio_s = scale_f16(weights["audio_embeddings.weight.s8"])
        self.projection = p("projection.weight")
        self.c0_head = p("codebook0_head.weight")
        self.audio_head = [p(f"audio_head.{i}") for i in range(N_CB - 1)]
        self.N = self.B = None

    def alloc(self, N, L, cfg_scale=1.5):
        self.N = N
        self.B = 2 * N if cfg_scale != 1.0 else N
        self.backbone.alloc(self.B, L)
        self.decoder.alloc(self.B, N_CB)

    def embed_audio(self, cb, tok):
        rows = np.asarray(tok, np.int64) + cb * AUDIO_VOCAB
        if self.audio_dense is not None:
            return self.audio_dense[rows]                    # F.embedding (app/engine.py:97)
        return K.embed_rows(self.audio_q8, self.audio_s, rows)

    def guided(self, logits, cfg, topk, temp, noise):
        N, B = self.N, self.B
        lg = cfg_mix(logits, N, cfg) if B == 2 * N else np.asarray(logits, np.float16)
        s = sample(lg.astype(np.float32), topk, temp, noise)
        return np.concatenate([s, s], 0) if B == 2 * N else s

    def frame(self, last_h, cfg=1.5, topk=50, temp=1.0, noise=None, forced=None):
        """_frame_fast (app/engine.py:328-343).  noise: [8, N, V] Exponential(1) draws;
        forced: [B, 8] tokens for teacher forcing (replace the samples).
        Returns (tokens [B, 8], logits list of 8 x [B, V] fp16)."""
        B = self.B
        logits = []

        def pick(i, lg):
            logits.append(lg)
            if forced is not None:
                return np.asarray(forced, np.int64)[:, i:i + 1]
            return self.guided(lg, cfg, topk, temp, noise[i])

        c0 = pick(0, self.c0_head(last_h))
        samples = [c0]
        x = np.stack([last_h, self.embed_audio(0, c0)[:, 0]], 1).reshape(2 * B, -1)
        dpos0 = np.tile(np.arange(2, dtype=np.int64), B)
        h = self._pair_last(self.decoder.decode(self.projection(x), dpos0, 2))
        for i in range(1, N_CB):
            ci = pick(i, self._audio_head(i)(h))
            samples.append(ci)
            if i < N_CB - 1:
                e = self.embed_audio(i, ci)[:, 0]
                h = self.decoder.decode(self.projection(e), np.full(B, self._dec_pos(i), np.int64), 1)
        return np.concatenate(samples, 1), logits

    # the three composition choices of _frame_fast, kept as methods so the pins in
    # tests/test_oracle_frame.py can show that a slip in any of them is caught
    @staticmethod
    def _pair_last(h):
        """Pass 0 runs rows (backbone state, codebook-0 embedding) per batch entry; the
        codebook-1 head reads the second row of each pair (app/engine.py:337, [1::2])."""
        return h[1::2]

    def _audio_head(self, i):
        """Codebook i (1..7) is read by audio_head[i - 1] (app/engine.py:339)."""
        return self.audio_head[i - 1]

    @staticmethod
    def _dec_pos(i):
        """Decoder position of the pass that embeds codebook i (app/engine.py:332, :342)."""
        return i + 1

    def step(self, tok, pos, **kw):
        """_step (app/engine.py:345-349): tok [B, 8] previous frame, pos scalar position."""
        if self.audio_dense is not None:
            rows = np.asarray(tok, np.int64) + np.arange(N_CB)[None] * AUDIO_VOCAB
            h = K.sum_rows(self.audio_dense[rows])
        else:
            h = K.embed_sum(self.audio_q8, self.audio_s, tok, AUDIO_VOCAB)
        last_h = self.backbone.decode(h, np.full(self.B, pos, np.int64), 1)
        return self.frame(last_h, **kw)


def frame_loop_trim(frames, n_frames, check=25, eos=8193):
    """The frame loop's EOS scan and per-take trim (app/engine.py:401-446) applied to a token
    sequence: frames [n_frames + 1, N, 8] (frame 0 from the prompt pass, frame i + 1 made by
    loop iteration i).  Every ``check`` iterations, and after the last, the frames since the
    previous check (never frame 0) are scanned for a token >= ``eos``; a take's end is its first
    such frame; the loop stops at the first check where every take has ended.  A take is
    trimmed to the frames before its end (all frames up to the last one made if it never
    ended).  Returns (list of N int64 arrays [8, T], loop iterations run)."""
    frames = np.asarray(frames, np.int64)
    N = frames.shape[1]
    ends = [None] * N
    last = n_frames
    ran = n_frames
    for i in range(n_frames):
        if (i + 1) % check == 0 or i == n_frames - 1:
            a = max(1, i + 2 - check)
            hit = (frames[a:i + 2] >= eos).any(-1)                    # [t, N]
            for c in range(N):
                if ends[c] is None and hit[:, c].any():
                    ends[c] = a + int(np.flatnonzero(hit[:, c])[0])
            if all(e is not None for e in ends):
                last = ran = i + 1
                break
    out = []
    for c in range(N):
        T = ends[c] if ends[c] is not None else last + 1
        out.append(frames[:T, c].T.copy())
    return out, ran
