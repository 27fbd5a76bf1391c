"""The codec's flow-matching estimator and Euler solver on gfx950.

Mirrors ``LlamaTransformer`` with ``norm_type="ada_norm_single"``
(app/heartcodec/models/transformer.py:275-396) and ``FlowMatching.solve_euler``
(app/heartcodec/models/flow_matching.py:161-210), run in fp16 as the reference loads the codec
(app/codec_lite.py:13,27).  Every step is a HIP kernel of ``libecdecode.so``:

    ProjectLayer (k = 3 conv + Linear)   ecd_codec_cols3 + ecd_gemm_f16p (x2)
    adaLN + RMSNorm / gated residual     ecd_codec_norm_mod
    q | k | v projection                 ecd_gemm_f16p (one GEMM, N = 3D)
    q | k | v linear + interleaved RoPE  ecd_gemm_f16p_rope (ecd_codec_rope_heads standalone)
    non-causal SDPA                      ecd_prefill_attn (every row at the last slot)
    LlamaMLP                             ecd_gemm_f16p_silu + ecd_gemm_f16p
    timestep path                        ecd_codec_timestep, ecd_gemm_f16p, ecd_codec_silu
    Euler + CFG + in-context blend       ecd_codec_euler

The solver computes the adaLN vectors of all steps in one batched pass before the loop (they
depend only on t), and feeds the estimator's [x | incontext | mu] input to the first
convolution as channel segments instead of concatenated copies.  There is no CPU fallback:
without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _ffi
from .kernels import (gemm_f16_packed, gemm_f16_silu_packed, pack_f16, prefill_attn,
                      stream_ptr)

__all__ = ["LlamaTransformer", "CodeEmbedding", "solve_euler", "inference_codes",
           "detokenize_latents", "detokenize", "crossfade_windows", "ScalarDecoder",
           "random_code_embedding_state_dict",
           "random_decoder_state_dict", "decoder_flops",
           "mlp_hidden",
           "euler_times", "t_span", "random_state_dict", "estimator_flops"]

EPS = 1e-6
SQRT1_3 = 3 ** -0.5


def mlp_hidden(dim: int, multiple_of: int = 256) -> int:
    """LlamaMLP hidden width (transformer.py:170-172)."""
    h = int(2 * (4 * dim) / 3)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


def euler_times(t_span) -> tuple[list[np.float32], list[np.float32]]:
    """The fp32 (t, dt) of every Euler step as solve_euler advances them (flow_matching.py:
    172-173, 204-207): t += dt, then dt = t_span[k + 1] - t."""
    ts = np.asarray(t_span, dtype=np.float32)
    t, dt = ts[0], np.float32(ts[1] - ts[0])
    out_t, out_dt = [], []
    for step in range(1, len(ts)):
        out_t.append(np.float32(t))
        out_dt.append(np.float32(dt))
        t = np.float32(t + dt)
        if step < len(ts) - 1:
            dt = np.float32(ts[step + 1] - t)
    return out_t, out_dt


def _off(t: torch.Tensor, elems: int) -> int:
    """Device address of element ``elems`` of a contiguous fp16 tensor."""
    return t.data_ptr() + 2 * int(elems)


class _Linear:
    """One nn.Linear (or a k = 3 Conv1d as a GEMM) with packed fp16 weights, fp32 bias."""

    def __init__(self, w: torch.Tensor, b: torch.Tensor | None = None, interleave=False):
        self.N, self.K = w.shape
        self.wp = pack_f16(w.contiguous(), interleave=interleave)
        self.b = None if b is None else b.float().contiguous()

    def __call__(self, x, out, alpha=1.0, res=None):
        return gemm_f16_packed(x, self.wp, self.N, self.K, self.b, alpha, res, out)


class _Block:
    """Weights of one LlamaTransformerBlock (transformer.py:184-255)."""

    def __init__(self, get, pre: str, dim: int, heads: int, head_dim: int):
        self.D, self.H, self.HD = dim, heads, head_dim
        self.qkv = _Linear(torch.cat([get(pre + "attn.q_proj.weight"),
                                      get(pre + "attn.k_proj.weight"),
                                      get(pre + "attn.v_proj.weight")], 0))
        self.o = _Linear(get(pre + "attn.o_proj.weight"))
        gate, up = get(pre + "mlp.gate.weight"), get(pre + "mlp.up.weight")
        self.F = gate.shape[0]
        self.gu = pack_f16(torch.cat([gate, up], 0).contiguous(), interleave=True)
        self.down = _Linear(get(pre + "mlp.down.weight"))
        self.attn_norm = get(pre + "attn_norm.weight")
        self.mlp_norm = get(pre + "mlp_norm.weight")
        self.table = get(pre + "scale_shift_table")        # [6, D]


class _Ada:
    """AdaLayerNormSingleFlow weights (transformer.py:429-458)."""

    def __init__(self, get, pre: str):
        te = pre + "emb.timestep_embedder."
        self.l1 = _Linear(get(te + "linear_1.weight"), get(te + "linear_1.bias"))
        self.l2 = _Linear(get(te + "linear_2.weight"), get(te + "linear_2.bias"))
        self.lin = _Linear(get(pre + "linear.weight"), get(pre + "linear.bias"))


class _Project:
    """ProjectLayer(kernel_size=3) weights (transformer.py:258-272): the conv as a GEMM over
    [t - 1 | t | t + 1] columns, W'[o, j * Cin + c] = weight[o, c, j]."""

    def __init__(self, get, pre: str):
        w = get(pre + "ffn_1.weight")                       # [Cout, Cin, 3]
        self.cout, self.cin, k = w.shape
        if k != 3:
            raise ValueError(f"{pre}ffn_1: kernel size {k}, expected 3")
        self.conv = _Linear(w.permute(0, 2, 1).reshape(self.cout, 3 * self.cin).contiguous(),
                            get(pre + "ffn_1.bias"))
        self.ffn_2 = _Linear(get(pre + "ffn_2.weight"), get(pre + "ffn_2.bias"))


class LlamaTransformer:
    """The estimator: ``forward(hidden_states, timestep)`` as in transformer.py:345-396.

    ``sd`` maps the reference's parameter names relative to the estimator
    (``proj_in.ffn_1.weight``, ``transformer_blocks.0.attn.q_proj.weight``, ...) to tensors;
    ``from_codec_state_dict`` takes a whole HeartCodec state dict."""

    def __init__(self, sd: dict, num_attention_heads=24, attention_head_dim=64, in_channels=1024,
                 out_channels=256, num_layers=24, num_layers_2=6, device="cuda"):
        self.dev = torch.device(device)
        if self.dev.type != "cuda":
            raise RuntimeError("the codec estimator runs only on a ROCm GPU")
        self.H, self.HD = num_attention_heads, attention_head_dim
        self.D = self.H * self.HD
        self.D2 = 2 * self.D
        self.cin, self.cout = in_channels, out_channels

        def get(name):
            return sd[name].to(device=self.dev, dtype=torch.float16).contiguous()

        self.proj_in = _Project(get, "proj_in.")
        self.blocks = [_Block(get, f"transformer_blocks.{i}.", self.D, self.H, self.HD)
                       for i in range(num_layers)]
        self.blocks_2 = [_Block(get, f"transformer_blocks_2.{i}.", self.D2, self.H, 2 * self.HD)
                         for i in range(num_layers_2)]
        self.connection_proj = _Project(get, "connection_proj.")
        self.proj_out = _Project(get, "proj_out.")
        self.table = get("scale_shift_table")               # [2, D]
        self.table_2 = get("scale_shift_table_2")           # [2, D2]
        self.ada = _Ada(get, "adaln_single.")
        self.ada_2 = _Ada(get, "adaln_single_2.")
        if (self.proj_in.cin, self.proj_in.cout) != (in_channels, self.D):
            raise ValueError("proj_in shape does not match the configuration")
        self._bufs = {}
        self._rope = {}

    @classmethod
    def from_codec_state_dict(cls, sd: dict, prefix="flow_matching.estimator.", **cfg):
        return cls({k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}, **cfg)

    # ------------------------------------------------------------ timestep path
    def timestep_vectors(self, t: torch.Tensor):
        """adaln_single / adaln_single_2 for every entry of t [n] fp32: (tmod [n, 6D],
        emb [n, D], tmod_2 [n, 6D2], emb_2 [n, D2]) (transformer.py:354-357, :377-380)."""
        t = t.to(device=self.dev, dtype=torch.float32).contiguous()
        n = t.numel()
        st = stream_ptr(self.dev)
        sin = torch.empty(n, 512, device=self.dev, dtype=torch.float16)
        _ffi.call("ecd_codec_timestep", t.data_ptr(), sin.data_ptr(), n, st)
        out = []
        for ada, D in ((self.ada, self.D), (self.ada_2, self.D2)):
            h = ada.l1(sin, torch.empty(n, D, device=self.dev, dtype=torch.float16))
            _ffi.call("ecd_codec_silu", h.data_ptr(), h.data_ptr(), h.numel(), st)
            emb = ada.l2(h, torch.empty(n, D, device=self.dev, dtype=torch.float16))
            se = torch.empty_like(emb)
            _ffi.call("ecd_codec_silu", emb.data_ptr(), se.data_ptr(), emb.numel(), st)
            tmod = ada.lin(se, torch.empty(n, 6 * D, device=self.dev, dtype=torch.float16))
            out += [tmod, emb]
        return tuple(out)

    # ------------------------------------------------------------ buffers
    def _buffers(self, B: int, T: int):
        """Work buffers for B sequences of T frames, cached for the latest shape only (a new
        shape releases the old buffers to torch's stream-ordered allocator)."""
        key = (B, T)
        if key not in self._bufs:
            self._bufs.clear()
            M, D2 = B * T, self.D2
            F2 = max(b.F for b in self.blocks + self.blocks_2)
            cmax = max(self.cin + self.D, D2, self.cin)
            e = lambda *s: torch.empty(*s, device=self.dev, dtype=torch.float16)
            self._bufs[key] = dict(
                cols=e(M * 3 * cmax), t1=e(M * D2), x=e(M * D2), y=e(M * D2),
                q=e(M * D2), k=e(M * D2), v=e(M * D2), o=e(M * D2), h=e(M * D2), m=e(M * F2),
                out=e(M, self.cout),
                pos=torch.full((M,), T - 1, device=self.dev, dtype=torch.int64))
        return self._bufs[key]

    def _rope_table(self, T: int, HD: int):
        key = (T, HD)
        if key not in self._rope:
            tab = torch.empty(T, HD, device=self.dev, dtype=torch.float16)
            _ffi.call("ecd_codec_rope_table", tab.data_ptr(), T, HD, stream_ptr(self.dev))
            self._rope[key] = tab
        return self._rope[key]

    # ------------------------------------------------------------ pieces
    def _cols(self, segs, B, T, buf):
        """k = 3 columns of the channel concatenation of ``segs`` [(tensor, width, bmod, bzero)
        or (tensor, width, bmod, bzero, rep)]; rep 2 reads a half-rate source upsampled 2x."""
        n = len(segs)
        rp = (ctypes.c_int * n)(*[s[4] if len(s) > 4 else 1 for s in segs])
        ptr = (ctypes.c_void_p * n)(*[s[0].data_ptr() for s in segs])
        ld = (ctypes.c_long * n)(*[s[0].stride(-2) for s in segs])
        w = (ctypes.c_int * n)(*[s[1] for s in segs])
        bm = (ctypes.c_int * n)(*[s[2] for s in segs])
        bz = (ctypes.c_int * n)(*[s[3] for s in segs])
        C = sum(s[1] for s in segs)
        cols = buf["cols"][:B * T * 3 * C].view(B * T, 3 * C)
        _ffi.call("ecd_codec_cols3", ptr, ld, w, bm, bz, rp, n, cols.data_ptr(), B, T,
                  stream_ptr(self.dev))
        return cols

    def _project(self, p: _Project, cols, buf):
        M = cols.shape[0]
        t1 = p.conv(cols, buf["t1"][:M * p.cout].view(M, p.cout), alpha=SQRT1_3)
        return t1

    def _norm(self, x, h, gate, w, shift, scale, tm_ld, y, T, norm):
        """gate/shift/scale: (table address, vector address); gate None: no residual."""
        R, D = x.shape
        g_tab, g_tm, g_ld = gate if gate is not None else (None, None, 0)
        _ffi.call("ecd_codec_norm_mod", x.data_ptr(), None if h is None else h.data_ptr(),
                  g_tab, g_tm, g_ld, None if w is None else w.data_ptr(), shift[0], shift[1],
                  scale[0], scale[1], tm_ld, y.data_ptr(), R, T, D, norm, EPS,
                  stream_ptr(self.dev))

    def _blocks(self, blocks, x, B, T, tmod, tm_ld, buf):
        """The LlamaTransformerBlock stack; returns the pending gated residual (h, gate) of the
        last block's MLP, which the following norm applies."""
        M = B * T
        h, gate = None, None
        st = stream_ptr(self.dev)
        for bp in blocks:
            D, H, HD = bp.D, bp.H, bp.HD
            ch = lambda i: (_off(bp.table, i * D), _off(tmod, i * D))
            y = buf["y"][:M * D].view(M, D)
            self._norm(x, h, None if gate is None else gate + (tm_ld,), bp.attn_norm, ch(0), ch(1),
                       tm_ld, y, T, 0)
            q = buf["q"][:M * D].view(M, D)
            k = buf["k"][:M * D].view(B, H, T, HD)
            v = buf["v"][:M * D].view(B, H, T, HD)
            # q | k | v projection with RoPE and the head layout in the GEMM epilogue
            _ffi.call("ecd_gemm_f16p_rope", y.data_ptr(), D, bp.qkv.wp.data_ptr(), None,
                      self._rope_table(T, HD).data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      M, T, H, HD, D, st)
            o = prefill_attn(q, k, v, buf["pos"][:M], T, H, H, out=buf["o"][:M * D].view(M, D))
            ha = bp.o(o, buf["h"][:M * D].view(M, D))
            g_a = ch(2) + (tm_ld,)
            self._norm(x, ha, g_a, bp.mlp_norm, ch(3), ch(4), tm_ld, y, T, 0)
            m = gemm_f16_silu_packed(y, bp.gu, bp.F, D, out=buf["m"][:M * bp.F].view(M, bp.F))
            h = bp.down(m, buf["h"][:M * D].view(M, D))
            gate = ch(5)
        return h, gate

    def _run(self, segs, B, T, tm):
        """Estimator body over input segments; tm = (tmod, emb, tmod_2, emb_2, per_batch)."""
        tmod, emb, tmod2, emb2, per_batch = tm
        buf = self._buffers(B, T)
        M, D, D2 = B * T, self.D, self.D2
        # proj_in
        cols = self._cols(segs, B, T, buf)
        t1 = self._project(self.proj_in, cols, buf)
        x = self.proj_in.ffn_2(t1, buf["x"][:M * D].view(M, D))
        h, gate = self._blocks(self.blocks, x, B, T, tmod, 6 * D if per_batch else 0, buf)
        # norm_out with the scale_shift_table modulation
        s = buf["o"][:M * D].view(M, D)
        e_ld = D if per_batch else 0
        self._norm(x, h, gate + (6 * D if per_batch else 0,), None,
                   (_off(self.table, 0), _off(emb, 0)), (_off(self.table, D), _off(emb, 0)),
                   e_ld, s, T, 1)
        # connection_proj over [hidden_states | s]
        cols = self._cols(segs + [(s, D, B, 0)], B, T, buf)
        t1 = self._project(self.connection_proj, cols, buf)
        x2 = self.connection_proj.ffn_2(t1, buf["x"][:M * D2].view(M, D2))
        h, gate = self._blocks(self.blocks_2, x2, B, T, tmod2, 6 * D2 if per_batch else 0, buf)
        s2 = buf["o"][:M * D2].view(M, D2)
        e_ld = D2 if per_batch else 0
        self._norm(x2, h, gate + (6 * D2 if per_batch else 0,), None,
                   (_off(self.table_2, 0), _off(emb2, 0)), (_off(self.table_2, D2), _off(emb2, 0)),
                   e_ld, s2, T, 1)
        cols = self._cols([(s2, D2, B, 0)], B, T, buf)
        t1 = self._project(self.proj_out, cols, buf)
        return self.proj_out.ffn_2(t1, buf["out"][:M])

    # ------------------------------------------------------------ reference entry point
    def forward(self, hidden_states: torch.Tensor, timestep: torch.Tensor) -> torch.Tensor:
        """hidden_states [B, T, in_channels] fp16, timestep [B] -> [B, T, out_channels] fp16
        (a new tensor)."""
        B, T, C = hidden_states.shape
        if C != self.cin or hidden_states.dtype != torch.float16 or not hidden_states.is_contiguous():
            raise ValueError(f"hidden_states must be contiguous fp16 [B, T, {self.cin}]")
        if timestep.numel() != B:
            raise ValueError("timestep must hold one value per batch entry")
        tm = self.timestep_vectors(timestep.reshape(-1)) + (True,)
        out = self._run([(hidden_states.view(B * T, C), C, B, 0)], B, T, tm)
        return out.view(B, T, self.cout).clone()

    __call__ = forward


def solve_euler(est: LlamaTransformer, x: torch.Tensor, incontext_x: torch.Tensor,
                incontext_length: int, t_span, mu: torch.Tensor, guidance_scale: float,
                copy_incontext: bool = False, mu_rep: int = 1) -> torch.Tensor:
    """FlowMatching.solve_euler (flow_matching.py:161-210) on the GPU.  x, incontext_x
    [B, T, C] fp16, mu [B, T / mu_rep, Cmu] fp16 (mu_rep 2: half-rate mu, read as its nearest
    2x upsampling), t_span the fp32 time grid.  Returns the final x (a new tensor).
    ``copy_incontext`` also applies inference_codes' final
    ``latents[:, :L] = incontext_latents[:, :L]`` (flow_matching.py:156-158)."""
    B, T, C = x.shape
    Cmu = mu.shape[-1]
    if C + C + Cmu != est.cin:
        raise ValueError("x, incontext_x and mu widths must add up to the estimator's input")
    if mu_rep not in (1, 2) or T % mu_rep or mu.shape[:2] != (B, T // mu_rep):
        raise ValueError("mu must be [B, T / mu_rep, Cmu] with mu_rep 1 or 2")
    for a in (x, incontext_x, mu):
        if a.dtype != torch.float16 or not a.is_contiguous() or a.shape[0] != B:
            raise ValueError("x, incontext_x, mu must be contiguous fp16 [B, T, *]")
    if x.shape != incontext_x.shape:
        raise ValueError("incontext_x must be shaped like x")
    L = int(incontext_length)
    ts, dts = euler_times(t_span)
    n = len(ts)
    cfg = guidance_scale > 1.0
    dev = est.dev
    st = stream_ptr(dev)
    tmod, emb, tmod2, emb2 = est.timestep_vectors(torch.tensor(np.array(ts, np.float32)))
    noise = x.clone()
    x = x.clone()
    ic = incontext_x
    B2 = 2 * B if cfg else B
    # rows of the estimator input: [x | incontext | 0 (uncond) or mu (cond)] over 2B entries
    segs = [(x.view(B * T, C), C, B, 0), (ic.view(B * T, C), C, B, 0),
            (mu.view(B * (T // mu_rep), Cmu), Cmu, B, B if cfg else 0, mu_rep)]
    _ffi.call("ecd_codec_euler", x.data_ptr(), noise.data_ptr(), ic.data_ptr(), None, int(cfg),
              B, T, C, L, 0.0, 0.0, float(ts[0]), 0, st)
    D, D2 = est.D, est.D2
    for k in range(n):
        tm = (tmod[k], emb[k], tmod2[k], emb2[k], False)
        d = est._run(segs, B2, T, tm)
        last = k == n - 1
        if last and copy_incontext:
            mode, tb = 1, 0.0
        else:
            mode, tb = 0, (0.0 if last else float(ts[k + 1]))
        _ffi.call("ecd_codec_euler", x.data_ptr(), noise.data_ptr(), ic.data_ptr(), d.data_ptr(),
                  int(cfg), B, T, C, 0 if (last and not copy_incontext) else L, float(dts[k]),
                  float(guidance_scale), tb, mode, st)
    return x


class CodeEmbedding:
    """The conditioning of FlowMatching.inference_codes (flow_matching.py:86-108): per-quantizer
    codebook rows summed (ResidualVQ.get_codes_from_indices + sum), ``project_out``,
    ``cond_feature_emb``.  Returns the half-rate features [B * Tc, dim]; the estimator input
    reads them through the nearest 2x upsampling (``solve_euler(..., mu_rep=2)``).

    ``sd`` maps the reference's names relative to ``flow_matching.`` (``vq_embed.layers.{q}.
    _codebook.embed`` [1, V, Dc], ``vq_embed.project_out.{weight,bias}``,
    ``cond_feature_emb.{weight,bias}``)."""

    def __init__(self, sd: dict, num_quantizers=8, device="cuda"):
        self.dev = torch.device(device)
        get = lambda n: sd[n].to(device=self.dev, dtype=torch.float16).contiguous()
        books = [get(f"vq_embed.layers.{q}._codebook.embed") for q in range(num_quantizers)]
        self.Q = num_quantizers
        self.V, self.Dc = books[0].shape[-2], books[0].shape[-1]
        self.books = torch.stack([b.reshape(self.V, self.Dc) for b in books]).contiguous()
        self.Wp = (self.Dc + 63) // 64 * 64          # K of the projection padded to the GEMM
        po = get("vq_embed.project_out.weight")      # [dim, Dc]
        self.dim = po.shape[0]
        pw = torch.zeros(self.dim, self.Wp, device=self.dev, dtype=torch.float16)
        pw[:, :self.Dc] = po
        self.project_out = _Linear(pw, get("vq_embed.project_out.bias"))
        self.cond = _Linear(get("cond_feature_emb.weight"), get("cond_feature_emb.bias"))

    def __call__(self, codes: torch.Tensor, clamp: bool = False) -> torch.Tensor:
        """codes [B, Q, Tc] int64 (any strides with unit stride along Tc) -> [B * Tc, dim].
        ``clamp``: codes clamped to [0, V - 1] first (codec_lite.decode); otherwise -1 and
        out-of-range codes contribute nothing (get_codes_from_indices' padding)."""
        B, Q, Tc = codes.shape
        if Q != self.Q or codes.dtype != torch.int64 or codes.stride(2) != 1:
            raise ValueError(f"codes must be int64 [B, {self.Q}, Tc] with unit stride in time")
        codes = codes.to(self.dev)
        st = stream_ptr(self.dev)
        e = torch.empty(B * Tc, self.Wp, device=self.dev, dtype=torch.float16)
        _ffi.call("ecd_codec_vq_embed", codes.data_ptr(), codes.stride(0), codes.stride(1),
                  self.books.data_ptr(), e.data_ptr(), B, Q, Tc, self.V, self.Dc, self.Wp,
                  int(clamp), st)
        h = self.project_out(e, torch.empty(B * Tc, self.dim, device=self.dev, dtype=torch.float16))
        return self.cond(h, torch.empty_like(h))


def t_span(num_steps: int) -> np.ndarray:
    """torch.linspace(0, 1, num_steps + 1) in fp32 (flow_matching.py:140-142), evaluated as
    torch's linspace does: the first half from the start, the second half from the end."""
    n = num_steps + 1
    step = np.float32(1.0) / np.float32(n - 1)
    i = np.arange(n, dtype=np.float32)
    lo = (step * i).astype(np.float32)
    hi = (np.float32(1.0) - (step * (np.float32(n - 1) - i)).astype(np.float32)).astype(np.float32)
    return np.where(np.arange(n) < n // 2, lo, hi).astype(np.float32)


def inference_codes(emb: CodeEmbedding, est: LlamaTransformer, codes: torch.Tensor,
                    true_latents: torch.Tensor, latent_length: int, incontext_length: int,
                    guidance_scale: float = 2.0, num_steps: int = 20, scenario: str = "start_seg",
                    noise: torch.Tensor | None = None, clamp: bool = False) -> torch.Tensor:
    """FlowMatching.inference_codes (flow_matching.py:72-159): codes [B, Q, Tc] -> latents
    [B, 2 Tc, latent_dim] fp16.  ``noise`` is the initial latent sample (the reference draws it
    with torch.randn on its global generator); drawn from torch's device generator when None.
    Every frame must be a conditioned frame (latent_length == 2 Tc), as in detokenize."""
    B, _, Tc = codes.shape
    T = 2 * Tc
    C = true_latents.shape[-1]
    if latent_length != T:
        raise NotImplementedError("frames past latent_length (zero_cond rows) are not built")
    dev = est.dev
    mu = emb(codes, clamp=clamp).view(B, Tc, emb.dim)
    x = (noise if noise is not None else torch.randn(B, T, C, device=dev)).to(
        device=dev, dtype=torch.float16).contiguous()
    L = int(incontext_length) if scenario == "other_seg" else 0
    ic = torch.zeros(B, T, C, device=dev, dtype=torch.float16)
    if L:
        ic[:, :L] = true_latents[:, :L].to(device=dev, dtype=torch.float16)
    return solve_euler(est, x, ic, L, t_span(num_steps), mu, guidance_scale,
                       copy_incontext=True, mu_rep=2)


def detokenize_latents(emb: CodeEmbedding, est: LlamaTransformer, codes: torch.Tensor,
                       duration: float = 29.76, num_steps: int = 10,
                       guidance_scale: float = 1.25, randn=None) -> list:
    """The latent half of HeartCodec.detokenize (modeling_heartcodec.py:57-167) with
    codec_lite.decode's clamp of the codes (app/codec_lite.py:71): codes [Q, Tc] -> the latents
    [1, 25 duration, latent_dim] of every overlapping window, each later window continuing the
    previous one's last frames in context.  ``randn(shape)`` draws each window's initial sample
    (the only draw that reaches the output: the reference's other draws are masked to zero).
    The waveform decoder that turns these latents into audio is ``ScalarDecoder`` (see
    ``detokenize``)."""
    dev = est.dev
    if randn is None:
        randn = lambda shape: torch.randn(*shape, device=dev)
    codes = codes.unsqueeze(0).to(dev)
    C = est.cout
    min_samples = int(duration * 12.5)
    hop = min_samples // 93 * 80
    ovlp_samples = min_samples - hop
    ovlp_frames = ovlp_samples * 2
    if codes.shape[-1] < min_samples:
        while codes.shape[-1] < min_samples:
            codes = torch.cat([codes, codes], -1)
        codes = codes[:, :, :min_samples]
    codes_len = codes.shape[-1]
    if (codes_len - ovlp_frames) % hop > 0:   # the reference tests with ovlp_frames here
        len_codes = math.ceil((codes_len - ovlp_samples) / float(hop)) * hop + ovlp_samples
        while codes.shape[-1] < len_codes:
            codes = torch.cat([codes, codes], -1)
        codes = codes[:, :, :len_codes]
    latent_length = int(duration * 25)
    out = []
    for sinx in range(0, codes.shape[-1] - hop + 1, hop):
        win = codes[:, :, sinx:sinx + min_samples].contiguous()
        noise = randn((1, latent_length, C))
        if sinx == 0 or ovlp_frames == 0:
            true_latent = torch.zeros(1, latent_length, C, device=dev, dtype=torch.float16)
            L = 0
        else:
            true_latent = torch.zeros(1, latent_length, C, device=dev, dtype=torch.float16)
            true_latent[:, :ovlp_frames] = out[-1][:, -ovlp_frames:]
            L = ovlp_frames
        out.append(inference_codes(emb, est, win, true_latent, latent_length, L, guidance_scale,
                                   num_steps, "other_seg", noise=noise, clamp=True))
    return out


def random_state_dict(num_attention_heads=24, attention_head_dim=64, in_channels=1024,
                      out_channels=256, num_layers=24, num_layers_2=6, device="cuda", seed=0):
    """Random fp16 estimator weights under the reference's names, drawn on the device (there are
    no checkpoints here).  Scales keep activations O(1) through the stack."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    D = num_attention_heads * attention_head_dim
    D2 = 2 * D
    sd = {}

    def rnd(*shape, scale):
        return (torch.randn(*shape, generator=g, device=dev) * scale).half()

    def lin(name, n, k, bias=True, gain=1.0):
        sd[name + ".weight"] = rnd(n, k, scale=gain / k ** 0.5)
        if bias:
            sd[name + ".bias"] = rnd(n, scale=0.02)

    def proj(name, cout, cin):
        sd[name + ".ffn_1.weight"] = rnd(cout, cin, 3, scale=cin ** -0.5)
        sd[name + ".ffn_1.bias"] = rnd(cout, scale=0.02)
        lin(name + ".ffn_2", cout, cout)

    def blk(pre, dim):
        sd[pre + "attn_norm.weight"] = (1 + rnd(dim, scale=0.1).float()).half()
        sd[pre + "mlp_norm.weight"] = (1 + rnd(dim, scale=0.1).float()).half()
        for nm in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin(pre + "attn." + nm, dim, dim, bias=False)
        F = mlp_hidden(dim)
        lin(pre + "mlp.gate", F, dim, bias=False)
        lin(pre + "mlp.up", F, dim, bias=False)
        lin(pre + "mlp.down", dim, F, bias=False)
        sd[pre + "scale_shift_table"] = rnd(6, dim, scale=dim ** -0.5)

    def ada(pre, dim):
        lin(pre + "emb.timestep_embedder.linear_1", dim, 512)
        lin(pre + "emb.timestep_embedder.linear_2", dim, dim)
        lin(pre + "linear", 6 * dim, dim, gain=0.5)

    proj("proj_in", D, in_channels)
    for i in range(num_layers):
        blk(f"transformer_blocks.{i}.", D)
    for i in range(num_layers_2):
        blk(f"transformer_blocks_2.{i}.", D2)
    proj("connection_proj", D2, in_channels + D)
    sd["scale_shift_table"] = rnd(2, D, scale=D ** -0.5)
    sd["scale_shift_table_2"] = rnd(2, D2, scale=D2 ** -0.5)
    proj("proj_out", out_channels, D2)
    ada("adaln_single.", D)
    ada("adaln_single_2.", D2)
    return sd


class _Conv:
    """One Conv1d (optionally weight-normed) as a GEMM over tap columns: W'[o, j*Cin + c] =
    weight[o, c, j], taps (j - k + 1) * dilation (causal) or j - (k - 1) / 2 (centred)."""

    def __init__(self, w, b, offsets, prelu=None):
        self.cout, self.cin, k = w.shape
        self.off = (ctypes.c_int * k)(*offsets)
        self.k = k
        self.lin = _Linear(w.permute(0, 2, 1).reshape(self.cout, k * self.cin).contiguous(), b)
        self.prelu = prelu


class _ConvT:
    """A causal ConvTranspose1d (kernel 2s, stride s, trailing s outputs dropped) as a GEMM over
    the tap columns [x[i], x[i - 1]]: output phase p of input step i is
    W[:, :, p]^T x[i] + W[:, :, p + s]^T x[i - 1], so W'[p*Cout + o, c] = weight[c, o, p],
    W'[p*Cout + o, Cin + c] = weight[c, o, p + s], and the [T, s*Cout] product is the upsampled
    [T*s, Cout] sequence."""

    def __init__(self, w, b, stride):
        self.cin, self.cout, k = w.shape
        if k != 2 * stride:
            raise ValueError("causal ConvTranspose1d needs kernel 2 * stride")
        self.s = stride
        wt = torch.cat([w[:, :, :stride], w[:, :, stride:]], 0)      # [2 Cin, Cout, s]
        wt = wt.permute(2, 1, 0).reshape(stride * self.cout, 2 * self.cin).contiguous()
        self.off = (ctypes.c_int * 2)(0, -1)
        self.k = 2
        self.prelu = None
        self.lin = _Linear(wt, b.repeat(stride))


class ScalarDecoder:
    """ScalarModel.decode (app/heartcodec/models/sq_codec.py:380-526) on the GPU, time-major:
    round(9 x) / 9 of the latent, a centred Conv1d (kernel 5), five ResDecoderBlocks (causal
    ConvTranspose1d upsampling, then five ResidualUnits: dilated causal conv -> PReLU -> 1x1
    conv -> PReLU -> + x), the PostProcessor (2x repeat, causal conv, PReLU) and a causal
    Conv1d to the waveform.  Weight-normed weights are folded once at load (ecd_codec_weight_norm).

    ``sd`` maps the reference's names relative to ``scalar_model.`` (``decoder.0.parametrizations.
    weight.original0`` / ``original1``, or ``weight_g`` / ``weight_v``; ``decoder.N.bias``, ...)."""

    ROWS_BYTES = 512 << 20      # tap-column chunk per GEMM call

    def __init__(self, sd: dict, latent_hidden_dim=128, init_channel=64,
                 upsample_factors=(5, 4, 4, 4, 3), upsample_kernel_sizes=(10, 8, 8, 8, 6),
                 default_kernel_size=7, delay_kernel_size=5, res_kernel_size=7, num_samples=2,
                 num_bands=1, device="cuda"):
        self.dev = torch.device(device)
        if num_samples != 2:
            raise NotImplementedError("the PostProcessor is built for num_samples 2")
        get = lambda n: sd[n].to(device=self.dev, dtype=torch.float16).contiguous()
        st = stream_ptr(self.dev)

        def wn(pre):
            """The folded weight of a weight-normed layer (or the plain weight)."""
            if pre + "weight" in sd:
                return get(pre + "weight")
            g = sd.get(pre + "parametrizations.weight.original0", sd.get(pre + "weight_g"))
            v = sd.get(pre + "parametrizations.weight.original1", sd.get(pre + "weight_v"))
            g = g.to(device=self.dev, dtype=torch.float16).contiguous()
            v = v.to(device=self.dev, dtype=torch.float16).contiguous()
            w = torch.empty_like(v)
            _ffi.call("ecd_codec_weight_norm", v.data_ptr(), g.data_ptr(), w.data_ptr(),
                      v.shape[0], v[0].numel(), st)
            return w

        def prelu(pre):
            return float(sd[pre + "weight"].float().reshape(-1)[0])

        k0 = delay_kernel_size
        self.latent_dim = latent_hidden_dim
        self.conv0 = _Conv(wn("decoder.0."), get("decoder.0.bias"),
                           [j - (k0 - 1) // 2 for j in range(k0)])
        self.blocks = []
        for i, s in enumerate(upsample_factors):
            pre = f"decoder.{1 + i}."
            up = _ConvT(wn(pre + "up_conv.layer."), get(pre + "up_conv.layer.bias"), s)
            if upsample_kernel_sizes[i] != 2 * s:
                raise ValueError("upsample kernel must be 2 * factor (causal)")
            if self.PAD % s:
                raise ValueError(f"upsampling factor {s} must divide the {self.PAD} pad rows")
            units = []
            for u, d in enumerate((1, 3, 5, 7, 9)):
                q = f"{pre}convs.{u}."
                kr = res_kernel_size
                c1 = _Conv(wn(q + "conv1."), get(q + "conv1.bias"),
                           [(j - kr + 1) * d for j in range(kr)], prelu(q + "activation1."))
                c2 = _Conv(wn(q + "conv2."), get(q + "conv2.bias"), [0], prelu(q + "activation2."))
                units.append((c1, c2))
            self.blocks.append((up, units))
        n_post = 1 + len(upsample_factors)
        kd = default_kernel_size
        causal = [j - kd + 1 for j in range(kd)]
        self.post = _Conv(get(f"decoder.{n_post}.conv.weight"), get(f"decoder.{n_post}.conv.bias"),
                          causal, prelu(f"decoder.{n_post}.activation."))
        self.final = _Conv(wn(f"decoder.{n_post + 1}."), get(f"decoder.{n_post + 1}.bias"), causal)
        self.num_bands = num_bands
        self._bufs = {}
        self._shape = None

    @classmethod
    def from_codec_state_dict(cls, sd: dict, prefix="scalar_model.", **cfg):
        return cls({k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}, **cfg)

    # Zero rows before each sequence of a padded activation: at least the widest causal reach
    # (6 taps at dilation 9 = 54) and divisible by every upsampling factor, so a transposed conv
    # writing s output rows per input row lands on the padded layout of the upsampled sequence.
    PAD = 60
    TAIL = 8     # zero rows after the last sequence

    def _pbuf(self, key, S, T, C):
        """Cached zero-padded time-major activation [S * (PAD + T) + TAIL, C].  The convolutions
        write only the data rows, so the padding stays zero across calls."""
        k = (key, S, T, C)
        if k not in self._bufs:
            self._bufs[k] = torch.zeros(S * (self.PAD + T) + self.TAIL, C, device=self.dev,
                                        dtype=torch.float16)
        return self._bufs[k]

    def _buf(self, key, rows, C):
        k = (key, rows, C)
        if k not in self._bufs:
            self._bufs[k] = torch.empty(rows, C, device=self.dev, dtype=torch.float16)
        return self._bufs[k]

    def _gemm(self, cv, x, ldx, M, T, xpad, taps, y, ldy, ypad, res=False, rep=1):
        """One conv as ecd_gemm_f16p_conv: implicit taps over the padded x (taps) or a plain x;
        rep = 2: x holds T / 2 rows per sequence, upsampled 2x by row repeat."""
        lin = cv.lin
        prelu = getattr(cv, "prelu", None)
        _ffi.call("ecd_gemm_f16p_conv", x.data_ptr(), ldx, lin.wp.data_ptr(),
                  lin.b.data_ptr() if lin.b is not None else None,
                  float(prelu) if prelu is not None else 1.0, y.data_ptr() if res else None,
                  ldy if res else 0, y.data_ptr(), ldy, M, lin.N, lin.K, T, xpad, ypad,
                  cv.off if taps else None, cv.k if taps else 0, rep, 2 if prelu is not None else 0,
                  stream_ptr(self.dev))

    def _cols_conv(self, cv, src, S, T, spad, rep, y, ypad):
        """A conv over materialised tap columns of src (padded by spad rows per sequence), its
        output rows written per sequence into y (padded by ypad rows), in chunks."""
        st = stream_ptr(self.dev)
        K = cv.lin.K
        C = K // cv.k
        step = max(256, self.ROWS_BYTES // (2 * K)) // 256 * 256
        cols = self._buf("cols", min(step, T), K)
        ld = y.stride(0)
        for b in range(S):
            for t0 in range(0, T, step):
                n = min(step, T - t0)
                c = cols[:n]
                _ffi.call("ecd_codec_cols_taps", src.data_ptr(), src.stride(0), cv.off, cv.k,
                          c.data_ptr(), S, T, C, rep, spad, b * T + t0, n, st)
                yr = y[b * (ypad + T) + ypad + t0:]
                self._gemm(cv, c, K, n, n, 0, False, yr, ld, -1)

    def decode(self, latent: torch.Tensor) -> torch.Tensor:
        """latent [1, T, S * latent_dim] fp16 (one window) -> waveform [S, T * up, num_bands]
        fp16, S = the channel groups (the two stereo channels), up = prod(factors) * 2."""
        _, T, W = latent.shape
        S = W // self.latent_dim
        if self._shape != (S, T):  # buffers are cached for the latest window shape only
            self._bufs.clear()
            self._shape = (S, T)
        st = stream_ptr(self.dev)
        P = self.PAD
        lat = latent.to(self.dev, torch.float16).contiguous()
        x0 = self._buf("lat", S * T, self.latent_dim)
        _ffi.call("ecd_codec_latent_split", lat.data_ptr(), x0.data_ptr(), T, S, self.latent_dim, st)
        a = self._pbuf("c0", S, T, self.conv0.cout)
        self._cols_conv(self.conv0, x0, S, T, 0, 1, a, P)
        for i, (up, units) in enumerate(self.blocks):
            s, C = up.s, up.cout
            bb = self._pbuf(f"b{i}", S, T * s, C)
            # transposed conv: GEMM rows are input steps, each writing s consecutive outputs
            self._gemm(up, a, up.cin, S * T, T, P, True, bb, s * C, P // s)
            T *= s
            h = self._buf(f"h{i}", S * T, C)
            for c1, c2 in units:
                self._gemm(c1, bb, C, S * T, T, P, True, h, C, -1)
                self._gemm(c2, h, C, S * T, T, 0, False, bb, C, P, res=True)
            a = bb
        T2 = 2 * T
        pb = self._pbuf("post", S, T2, self.post.cout)
        # PostProcessor: 2x row repeat + causal conv, read straight from the padded activation
        self._gemm(self.post, a, self.post.cin, S * T2, T2, P, True, pb, self.post.cout, P, rep=2)
        y = self._buf("out", S * T2, self.final.cout)
        self._gemm(self.final, pb, self.post.cout, S * T2, T2, P, True, y, self.final.cout, -1)
        return y.view(S, T2, -1).clone()


def crossfade_windows(windows: list, duration: float, sample_rate: int, target_len: int) -> np.ndarray:
    """The audio assembly of HeartCodec.detokenize (modeling_heartcodec.py:168-204), a host step in
    the reference too (each window is moved to the CPU first): every window [S, >= duration * sr]
    is cut to duration * sr samples, consecutive windows overlap by (min - min // 93 * 80) samples
    blended with a linear ramp in float64 and stored back in fp16 (through fp32, as torch's CPU
    copy rounds), the result cut to ``target_len``."""
    min_samples = int(duration * sample_rate)
    hop = min_samples // 93 * 80
    ovlp = min_samples - hop
    out = None
    for w in windows:
        cur = np.asarray(w, dtype=np.float16)[:, :min_samples]
        if out is None:
            out = cur
        elif ovlp == 0:
            out = np.concatenate([out, cur], -1)
        else:
            ramp = np.linspace(0, 1, ovlp)
            win = np.concatenate([ramp, 1 - ramp])
            mix = out[:, -ovlp:].astype(np.float64) * win[-ovlp:] + cur[:, :ovlp].astype(np.float64) * win[:ovlp]
            out = out.copy()
            out[:, -ovlp:] = mix.astype(np.float32).astype(np.float16)
            out = np.concatenate([out, cur[:, ovlp:]], -1)
    return out[:, :target_len]


def detokenize(emb: CodeEmbedding, est: LlamaTransformer, dec: ScalarDecoder, codes: torch.Tensor,
               duration: float = 29.76, num_steps: int = 10, guidance_scale: float = 1.25,
               sample_rate: int = 48000, randn=None) -> np.ndarray:
    """HeartCodec.detokenize (modeling_heartcodec.py:57-204) after codec_lite.decode's clamp:
    codes [Q, Tc] -> waveform [S, Tc / 12.5 * sample_rate] (fp16 numpy, on the host as the
    reference returns it).  Latents and waveform windows are computed on the GPU."""
    target_len = int(codes.shape[-1] / 12.5 * sample_rate)
    lat = detokenize_latents(emb, est, codes, duration, num_steps, guidance_scale, randn)
    wins = [dec.decode(l)[..., 0].cpu().numpy() for l in lat]
    return crossfade_windows(wins, duration, sample_rate, target_len)


def random_code_embedding_state_dict(num_quantizers=8, codebook_size=8192, codebook_dim=32,
                                     dim=512, device="cuda", seed=0):
    """Random fp16 code-embedding weights under the reference's names (relative to
    ``flow_matching.``), drawn on the device."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape, scale: (torch.randn(*shape, generator=g, device=dev) * scale).half()
    sd = {f"vq_embed.layers.{q}._codebook.embed": rnd(1, codebook_size, codebook_dim, scale=0.5)
          for q in range(num_quantizers)}
    sd["vq_embed.project_out.weight"] = rnd(dim, codebook_dim, scale=codebook_dim ** -0.5)
    sd["vq_embed.project_out.bias"] = rnd(dim, scale=0.02)
    sd["cond_feature_emb.weight"] = rnd(dim, dim, scale=dim ** -0.5)
    sd["cond_feature_emb.bias"] = rnd(dim, scale=0.02)
    sd["zero_cond_embedding1"] = rnd(dim, scale=1.0)
    return sd


def random_decoder_state_dict(latent_hidden_dim=128, init_channel=64,
                              upsample_factors=(5, 4, 4, 4, 3), device="cuda", seed=0):
    """Random fp16 waveform-decoder weights under the reference's names (relative to
    ``scalar_model.``; weight-normed layers as parametrization pairs), drawn on the device."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape, scale=1.0: (torch.randn(*shape, generator=g, device=dev) * scale).half()
    sd = {}
    ch = lambda i: init_channel * 2 ** (len(upsample_factors) - i)

    def wnl(pre, shape, fan):
        v = rnd(*shape)
        sd[pre + "parametrizations.weight.original1"] = v
        nrm = v.float().reshape(shape[0], -1).norm(dim=1)
        sd[pre + "parametrizations.weight.original0"] = (nrm / fan ** 0.5).half().reshape(-1, 1, 1)

    wnl("decoder.0.", (ch(0), latent_hidden_dim, 5), latent_hidden_dim * 5)
    sd["decoder.0.bias"] = rnd(ch(0), scale=0.02)
    for i, s in enumerate(upsample_factors):
        pre = f"decoder.{1 + i}."
        wnl(pre + "up_conv.layer.", (ch(i), ch(i + 1), 2 * s), ch(i) * 2)
        sd[pre + "up_conv.layer.bias"] = rnd(ch(i + 1), scale=0.02)
        c = ch(i + 1)
        for u in range(5):
            q = f"{pre}convs.{u}."
            wnl(q + "conv1.", (c, c, 7), c * 7 * 4)
            sd[q + "conv1.bias"] = rnd(c, scale=0.02)
            wnl(q + "conv2.", (c, c, 1), c * 4)
            sd[q + "conv2.bias"] = rnd(c, scale=0.02)
            sd[q + "activation1.weight"] = torch.full((1,), 0.25, device=dev).half()
            sd[q + "activation2.weight"] = torch.full((1,), 0.25, device=dev).half()
    n = 1 + len(upsample_factors)
    sd[f"decoder.{n}.conv.weight"] = rnd(init_channel, init_channel, 7, scale=(init_channel * 7) ** -0.5)
    sd[f"decoder.{n}.conv.bias"] = rnd(init_channel, scale=0.02)
    sd[f"decoder.{n}.activation.weight"] = torch.full((1,), 0.25, device=dev).half()
    wnl(f"decoder.{n + 1}.", (1, init_channel, 7), init_channel * 7)
    sd[f"decoder.{n + 1}.bias"] = rnd(1, scale=0.02)
    return sd


def decoder_flops(dec: ScalarDecoder, T: int, S: int = 2) -> int:
    """Algorithmic FLOPs of ScalarDecoder.decode on a [1, T, S * latent] window (2 M N K per
    conv as a GEMM, M = output rows)."""
    fl = 2 * S * T * dec.conv0.lin.N * dec.conv0.lin.K
    for up, units in dec.blocks:
        fl += 2 * S * T * up.lin.N * up.lin.K
        T *= up.s
        for c1, c2 in units:
            fl += 2 * S * T * (c1.lin.N * c1.lin.K + c2.lin.N * c2.lin.K)
    T *= 2
    fl += 2 * S * T * (dec.post.lin.N * dec.post.lin.K + dec.final.lin.N * dec.final.lin.K)
    return fl


def estimator_flops(est: LlamaTransformer, B: int, T: int) -> dict:
    """Algorithmic FLOPs of one estimator call on B x T rows: the dense layers (2 M N K each,
    the k = 3 convolutions as GEMMs with K = 3 Cin) and the attention products (4 B H T^2 HD per
    block: Q K^T and P V)."""
    M = B * T
    gemm = 0
    for p in (est.proj_in, est.connection_proj, est.proj_out):
        gemm += 2 * M * p.cout * 3 * p.cin + 2 * M * p.cout * p.cout
    attn = 0
    for bp in est.blocks + est.blocks_2:
        D, F = bp.D, bp.F
        gemm += 2 * M * (3 * D * D + D * D + 2 * F * D + D * F)
        attn += 4 * B * bp.H * T * T * bp.HD
    return {"gemm": gemm, "attn": attn, "total": gemm + attn}
