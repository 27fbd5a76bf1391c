"""HeartMuLa decode engine on gfx950: int8 weights, static KV cache, HIP kernels, hipGraphs.

Mirrors the fast path of the reference engine (app/engine.py) with the same classes,
method names and tensor layouts -- ``Linear``, ``fuse``, ``Emb``, ``Block``, ``Stack``
(``alloc``/``free``/``__call__``/``decode``) and ``HeartMuLaLite`` (``_embed_audio``,
``_frame_fast``, ``_step``, ``generate``, ``_capture``, ``release``) -- but every op of the
per-frame step is a hand-written HIP kernel reached through the C ABI of ``libecdecode.so``
(see ``kernels.py``), sampling included: one fused CFG + top-k + Exponential-race kernel per
codebook replaces the reference's ``_sample``/``_guided`` torch ops.  Differences from the
reference, all deliberate:

* stacks are shape-parametric (``dim`` per stack) instead of the global ``DIM = 3072``
  (app/engine.py:19, :116, :161), so a 1024-wide decoder can be expressed;
* the prompt pass (``Stack.__call__``) runs the MFMA GEMM and causal flash-attention kernels
  (more than 64 rows) or the decode kernels with one row per prompt position, instead of
  SDPA with ``repeat_interleave``; ``int8_mm`` keeps the reference's dense numerics for
  M > 16 rows;
* the prompt arrives as token ids (tokenisation is host string work, out of scope);
* the text-embedding table lives on the GPU (one gather per song);
* decode attention over caches of at most 128 slots uses one split (direct output,
  no combine pass); longer caches run the split attention and its merge in one launch,
  with enough splits to cover the CUs (``attention_kb``), where the reference launches 16
  splits and a combine; the reference's launch pair is kept for the drop-in path
  (``decode_reference``);
* the song loop keeps its bookkeeping on the device: the captured frame ends with a kernel
  that feeds the tokens back, stores the frame and records each take's first EOS frame, so
  the host only replays the graph and reads N integers every 25 frames.
"""
from __future__ import annotations

import json
import math
import warnings
from pathlib import Path

import torch

from . import _ffi
from .kernels import (_attn, _attn_combine, _rope_cache, _silu_mul, cdiv, embed_gemv_packed,
                      gemm_packed, gemm_silu_packed, gemv_packed_splitk, prefill_attn,
                      gemm_rope_packed, gemv_packed, int8_mm, layer_head, layer_stack,
                      layer_stack_plan, layer_stack_supported, layer_tail, layer_tail_supported,
                      layer_tail_ws_bytes, next_power_of_2,
                      pack_i8, rms as krms, rms_gemv_packed, rms_qkv_rope, rms_qkv_rope_rows,
                      rms_w13_silu,
                      sample_topk, stream_ptr)

AUDIO_VOCAB = 8197
PROMPT_GEMM_ROWS = 64  # prompt passes with more rows run the MFMA GEMM path
N_CB = 8
MUQ_DIM = 512
DIM = 3072
TEXT_BOS, TEXT_EOS, AUDIO_EOS, EMPTY_ID = 128000, 128001, 8193, 0
FRAME_MS = 80

ATT_SHORT = 128      # caches of at most this many slots: one attention split per (row, kv head)
ATT_WG = 256        # workgroups the merged attention grid aims at (one per CU of an MI355X)
ATT_KB_MAX = 16     # workgroups per (row, kv head) pair at most (the last one merges them all)
STACK_MAX = 64      # layers of one ecd_layer_stack launch at most
DECODER_RESIDENT = 160 << 20  # weight bytes of a decoder pass kept in the 256 MB Infinity Cache


def _overlap(a, b):
    """True when the storage of tensors a and b overlaps."""
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


def attention_kb(R, Hk, L):
    """Workgroups per (row, kv head) pair of the engine's decode attention over a cache of L
    slots (ecd_decode_attn_merged, 8 splits per workgroup): enough that R x Hk x kb workgroups
    cover the CUs and no split is longer than 128 slots, but no split shorter than one 16-slot
    tile and at most ATT_KB_MAX (measured on MI355X, 24q / 8kv, head_dim 128: one row at 4096
    slots takes 11.1 us with 16 workgroups per pair against 12.7 with 32; batch 8 takes
    31.7 us with 4 against 34.0 with 8, and 58.8 us at 8192 slots with 8 against 60.0 with 4)."""
    want = max(-(-ATT_WG // max(1, R * Hk)), -(-L // 1024))
    return max(1, min(ATT_KB_MAX, want, -(-L // 128)))


BACKBONE = dict(layers=28, heads=24, kv_heads=8, max_seq=8192, dim=DIM)
# the reference's depth decoder (app/engine.py:24; head_dim = 3072 // 8 = 384)
DECODER = dict(layers=3, heads=8, kv_heads=4, max_seq=2048, dim=DIM)
# the 1024-wide 4-layer decoder shape of the benchmark configuration
DECODER_1024 = dict(layers=4, heads=8, kv_heads=2, max_seq=2048, dim=1024)


# ---------------------------------------------------------------- RoPE (Llama-3 scaled)
def rope_cache(head_dim: int, max_seq: int, base=500_000, scale=32, low=1, high=4, old=8192,
               device="cuda"):
    """[max_seq, head_dim / 2, 2] float32 (cos, sin) built on the GPU (app/engine.py:28-43)."""
    dev = torch.device(device)
    out = torch.empty(max_seq, head_dim // 2, 2, device=dev, dtype=torch.float32)
    _ffi.call("ecd_rope_table", out.data_ptr(), max_seq, head_dim, float(base), float(scale),
              float(low), float(high), float(old), stream_ptr(dev))
    return out


# ---------------------------------------------------------------- linear layers
class Linear:
    """int8 per-output-channel linear layer (app/engine.py:62-79)."""

    def __init__(self, w=None, q8=None, s8=None):
        if q8 is None:
            raise NotImplementedError("the gfx950 decode path runs int8 per-channel weights only")
        self.w, self.q8, self.s8 = None, q8, s8
        self.qp = self.sp = None
        self.N, self.K = q8.shape
        self.stream = False
        self.ks = 1

    def pack(self, interleave=False, stream=False):
        """Add the lane-ordered tile copy used by the fused GEMVs (K % 64 == 0).  With
        ``interleave`` the w1 | w3 halves become (a_j, b_j) row pairs (scales likewise).
        ``stream``: the layer is read once per frame, so its loads bypass cache allocation."""
        self.stream = stream
        if self.K % 64:
            return self
        self.qp = pack_i8(self.q8, interleave)
        # few output tiles over a long K: split K over 4 workgroups per tile
        if (self.N + 15) // 16 <= 64 and self.K >= 4096 and (self.K // 64) % 4 == 0:
            self.ks = 4
        if interleave:
            F = self.N // 2
            self.sp = torch.stack([self.s8[:F], self.s8[F:]], 1).reshape(-1).contiguous()
        else:
            self.sp = self.s8
        return self

    def __call__(self, x, res=None):
        if self.qp is not None and self.sp is self.s8 and x.dim() == 2 and x.stride(1) == 1 \
                and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0:
            if self.ks > 1:
                return gemv_packed_splitk(x, self.qp, self.s8, self.N, self.K, self.ks, res,
                                          stream=self.stream)
            return gemv_packed(x, self.qp, self.s8, self.N, self.K, res, stream=self.stream)
        return int8_mm(x, self.q8, self.s8, res)

    @property
    def nbytes(self):
        return self.q8.numel() + self.s8.numel() * 2


def fuse(parts):
    """Row-concatenate layers that read the same input (q|k|v, w1|w3), app/engine.py:82-86."""
    return Linear(q8=torch.cat([p.q8 for p in parts]).contiguous(),
                  s8=torch.cat([p.s8 for p in parts]).contiguous())


class Emb:
    """Embedding table (app/engine.py:89-104): int8 rows with per-row fp16 scales, or dense fp16
    rows (the bf16 tables of a file written with --keep-emb-bf16, app/convert_final.py:43)."""

    def __init__(self, w=None, q8=None, s8=None):
        if w is None and q8 is None:
            raise ValueError("Emb needs a dense table w or int8 rows q8 with scales s8")
        if w is not None:
            if w.dtype != torch.float16:
                raise TypeError("Emb: the dense table must be float16 (the engine's dtype)")
            self.w, self.q8, self.s8 = w.contiguous(), None, None
        else:
            self.w, self.q8, self.s8 = None, q8.contiguous(), s8.contiguous()

    @property
    def table(self):
        return self.w if self.w is not None else self.q8

    @property
    def scales(self):
        """Per-row scales, or None for a dense fp16 table (the kernels' convention)."""
        return self.s8

    def _args(self):
        t = self.table
        return t.data_ptr(), (self.s8.data_ptr() if self.s8 is not None else None), t.shape[0]

    def __call__(self, idx):
        """The rows idx -> [*idx.shape, D] fp16."""
        idx = idx.to(torch.int64).contiguous()
        D = self.table.shape[1]
        out = torch.empty(*idx.shape, D, device=self.table.device, dtype=torch.float16)
        n = idx.numel()
        if n:
            tab, sc, rows = self._args()
            _ffi.call("ecd_embed_i8", idx.data_ptr(), 1, tab, sc, rows, 0, rows, None,
                      out.data_ptr(), n, D, stream_ptr(out.device))
        return out

    def gather(self, tok, cb, vocab, even=None):
        """One codebook: rows tok[:, 0] + cb * vocab -> [B, D]; with ``even`` [B, D] the result
        is the interleave [2B, D] (even rows = even, odd rows = embeddings)."""
        B = tok.shape[0]
        D = self.table.shape[1]
        out = torch.empty((2 * B if even is not None else B), D, device=self.table.device,
                          dtype=torch.float16)
        tab, sc, rows = self._args()
        _ffi.call("ecd_embed_i8", tok.data_ptr(), tok.stride(0), tab, sc, rows, int(cb), int(vocab),
                  even.data_ptr() if even is not None else None, out.data_ptr(), B, D,
                  stream_ptr(out.device))
        return out

    def sum_codebooks(self, tok, vocab):
        """sum_c Emb(tok[:, c] + c * vocab) accumulated in fp32, one fp16 rounding (:348)."""
        tok = tok.contiguous()
        B, C = tok.shape
        D = self.table.shape[1]
        out = torch.empty(B, D, device=self.table.device, dtype=torch.float16)
        tab, sc, rows = self._args()
        _ffi.call("ecd_embed_sum_i8", tok.data_ptr(), tab, sc, rows, out.data_ptr(), B, C, D,
                  int(vocab), stream_ptr(out.device))
        return out

    @property
    def nbytes(self):
        if self.w is not None:
            return self.w.numel() * 2
        return self.q8.numel() + self.s8.numel() * 2


# ---------------------------------------------------------------- static-cache transformer
class Block:
    def __init__(self, p, pre, heads, kv_heads, dim=DIM):
        self.qkv = fuse([p(pre + f"attn.{n}_proj.weight") for n in ("q", "k", "v")])
        self.o = p(pre + "attn.output_proj.weight")
        self.w13 = fuse([p(pre + "mlp.w1.weight"), p(pre + "mlp.w3.weight")])
        self.w2 = p(pre + "mlp.w2.weight")
        self.n1, self.n2 = p(pre + "sa_norm.scale", norm=True), p(pre + "mlp_norm.scale", norm=True)
        self.h, self.kvh = heads, kv_heads
        self.hd = dim // heads
        self.kc = self.vc = None

    def alloc(self, B, L, dev, dtype):
        self.kc = torch.zeros(B, self.kvh, L, self.hd, device=dev, dtype=dtype)
        self.vc = torch.zeros_like(self.kc)


class Stack:
    def __init__(self, p, prefix, cfg):
        dim = cfg.get("dim", DIM)
        self.blocks = [Block(p, f"{prefix}.layers.{i}.", cfg["heads"], cfg["kv_heads"], dim)
                       for i in range(cfg["layers"])]
        self.norm = p(f"{prefix}.norm.scale", norm=True)
        self.rope = None
        self.dim = dim
        self.hd = dim // cfg["heads"]
        self.max_seq = cfg["max_seq"]
        self.att_ws = None   # workgroup partials of the standalone attention (fp32)
        self.att_cnt = None  # its per-(row, kv head) counters (zero between calls)
        self.tail = None   # layer-tail buffers for B-row decode steps
        self.tail2 = None  # the same for 2B rows (two rows per cache), sharing sync, ws and err
        self.use_tail = True
        self.tail_attention = True  # the next layer's attention inside the tail launch
        self.tail_no_wait = False   # tests of the error path: every wait in the launches gives up
        self.tail_kv_nt = False     # the launches' attention reads every cache slot nontemporal
        self.use_stack = True       # all layer tails of a decode step as one launch where supported

    def alloc(self, B, L, dev, dtype):
        self.rope = rope_cache(self.hd, max(L, 16), device=dev)
        for b in self.blocks:
            b.alloc(B, L, dev, dtype)
        if self.blocks and L > ATT_SHORT:
            # partials of a decode step of up to 2B rows (two rows per cache) or of a short
            # prompt through the decode path (at most PROMPT_GEMM_ROWS rows): R rows take
            # R x Hk x attention_kb(R) workgroups of G head partials, at most ATT_KB_MAX R Hq
            hq, hk = max(b.h for b in self.blocks), max(b.kvh for b in self.blocks)
            rmax = max(2 * B, PROMPT_GEMM_ROWS)
            n = ATT_KB_MAX * rmax * hq
            self.att_ws = torch.empty(n * (2 + self.hd), device=dev, dtype=torch.float32)
            self.att_cnt = torch.zeros(rmax * hk, device=dev, dtype=torch.int32)
        self.tail = self._tail_buffers(B, dev, dtype, L)
        self.tail2 = None if self.tail is None else \
            self._tail_buffers(2 * B, dev, dtype, L, share=self.tail)

    def _tail_buffers(self, M, dev, dtype, L, share=None):
        """Static buffers of the one-launch layer tail (ecd_layer_tail) for M-row decode steps,
        or None when the shapes or weights do not fit it: x1, mm, two layer outputs used in
        turn (a launch's output never aliases its input), q, the gate region, the error
        word and the workspace (all three kept across launches)."""
        if not self.blocks or any(b.qkv.qp is None or b.o.qp is None or b.w13.qp is None or
                                  b.w2.qp is None for b in self.blocks):
            return None
        b0 = self.blocks[0]
        F = b0.w2.K
        if dtype != torch.float16 or not layer_tail_supported(M, self.dim, F, b0.h, b0.kvh, b0.hd):
            return None
        e = lambda n: torch.empty(M, n, device=dev, dtype=dtype)  # noqa: E731
        wsb = layer_tail_ws_bytes(self.dim, b0.h, b0.kvh, b0.hd)
        # the next layer's attention inside the launch (its output in one of two buffers)
        att = layer_tail_supported(M, self.dim, F, b0.h, b0.kvh, b0.hd, L, attention=True)
        if share is not None:  # launches in turn on one stream: one gate region and workspace
            sync, err, ws = share["sync"], share["err"], share["ws"]
        else:
            sync = torch.zeros(4096, device=dev, dtype=torch.int32)
            err = torch.zeros(1, device=dev, dtype=torch.int32)
            ws = torch.zeros(-(-wsb // 4), device=dev, dtype=torch.float32)
        t = dict(M=M, x1=e(self.dim), mm=e(F), xb=[e(self.dim), e(self.dim)],
                 q=e(b0.h * b0.hd), sync=sync, err=err, ws=ws,
                 att=att, ob=[e(b0.h * b0.hd), e(b0.h * b0.hd)] if att else None, plan=None)
        L0 = b0.kc.shape[2]
        stream = b0.w13.stream
        if att and len(self.blocks) <= STACK_MAX and any(
                layer_stack_supported(len(self.blocks), M, self.dim, F, b0.h, b0.kvh, b0.hd, L0,
                                      stream, nt)
                for nt in (False, True)):
            self._stack_buffers(t, M, F, dev, dtype)
        return t

    def _stack_buffers(self, t, M, F, dev, dtype):
        """Buffers and plan of the one-launch layer stack (ecd_layer_stack): every layer its own
        x1, mm, output and attention output (a launch writes no buffer twice), the records of
        the layers in a device plan."""
        nl, b0 = len(self.blocks), self.blocks[0]
        ew = lambda n: torch.empty(nl, M, n, device=dev, dtype=dtype)  # noqa: E731
        t["stack"] = dict(x1=ew(self.dim), mm=ew(F), xs=ew(self.dim), obs=ew(b0.h * b0.hd))
        t["plan"] = layer_stack_plan(self._stack_records(t), M, self.dim, F, b0.h, b0.kvh, b0.hd,
                                     dev)
        t["hplans"] = {}

    def _stack_records(self, t):
        """The layer records of a stack plan over the buffers of t["stack"]."""
        st, nl = t["stack"], len(self.blocks)
        layers = []
        for i, b in enumerate(self.blocks):
            nb = self.blocks[i + 1] if i + 1 < nl else None
            rec = dict(wo=b.o.qp, so=b.o.s8, n2=b.n2, w13=b.w13.qp, s13=b.w13.sp, w2=b.w2.qp,
                       s2=b.w2.s8, x1=st["x1"][i], mm=st["mm"][i], xout=st["xs"][i])
            if nb is not None:
                rec.update(n1=nb.n1, wq=nb.qkv.qp, sq=nb.qkv.s8, kc=nb.kc, vc=nb.vc,
                           o_next=st["obs"][i])
            layers.append(rec)
        return layers

    def head_plans(self, heads):
        """Stack plans that end in a codebook head: ``heads`` maps an index to (packed head
        Linear, logits buffer [M, N] with 16-byte aligned rows; M selects the buffers of B or 2B
        rows).  The last layer's record then runs rms(xout, stack norm) -> head GEMV into the
        buffer (the 1024-wide decoder; other stacks keep the head as its own launch).  Used by
        decode_head."""
        if self.dim != 1024:
            return
        b0, F = self.blocks[0], self.blocks[0].w2.K
        for i, (hd, y) in heads.items():
            t = next((t for t in (self.tail, self.tail2)
                      if t is not None and t["M"] == y.shape[0]), None)
            if t is None or t.get("plan") is None:
                continue
            layers = self._stack_records(t)
            layers[-1].update(n1=self.norm, wq=hd.qp, sq=hd.s8, y=y)
            t["hplans"][i] = (layer_stack_plan(layers, t["M"], self.dim, F, b0.h, b0.kvh, b0.hd,
                                               y.device), y)

    def decode_head(self, x, pos, S, head, o0=None):
        """One decode step whose last layer ends in codebook head ``head`` (head_plans): the
        logits buffer of that head, or None when the step cannot run as such a stack launch
        (the caller then runs decode and the head GEMV)."""
        R = x.shape[0]
        t = next((t for t in (self.tail, self.tail2) if t is not None and R == t["M"]), None)
        if t is None or head not in t.get("hplans", {}) or not self.use_tail:
            return None
        return self._decode_tail(x, pos, S, t, o0, head=head)

    def tail_error(self):
        """The error word of this stack's layer-tail launches (host sync): nonzero if one timed
        out waiting (bit 0, and one bit per wait that gave up, as include/ecdecode.h lists)."""
        return 0 if self.tail is None else int(self.tail["err"].item())

    def tail_reset(self):
        """Zero the launches' gate region, workspace and error word (after a timeout their
        contents are undefined)."""
        if self.tail is not None:
            for k in ("sync", "ws", "err"):
                self.tail[k].zero_()

    def free(self):
        for b in self.blocks:
            b.kc = b.vc = None
        self.tail = self.tail2 = self.att_ws = self.att_cnt = None

    def __call__(self, x, pos, attn_len=None, mask=None):
        """Prompt pass (app/engine.py:174-178): x [B, S, D], pos [B, S] absolute positions
        (causal).  Runs the decode kernels with one row per position; row (b, s) attends
        [0, pos[b, s]], which is the causal mask of the reference's SDPA call."""
        if mask is not None:
            raise NotImplementedError("explicit attention masks are not part of the fast path")
        B, S, D = x.shape
        x2 = x.reshape(B * S, D)
        p2 = pos.reshape(B * S).to(torch.int64).contiguous()
        if B * S > PROMPT_GEMM_ROWS and all(b.qkv.qp is not None for b in self.blocks):
            h = self._prompt_pass(x2.contiguous(), p2, S)
        else:
            h = self.decode(x2, p2, S)
        return h.reshape(B, S, D)

    def _prompt_pass(self, x, pos, S):
        """Many rows (app/engine.py:123-153): every Linear runs the MFMA GEMM with the
        reference's dense numerics (M > 16); RMSNorm, RoPE + cache write and the causal
        attention (row r attends [0, pos[r]]) use the decode kernels."""
        R = x.shape[0]
        for b in self.blocks:
            Hq, Hk, HD, L = b.h, b.kvh, b.hd, b.kc.shape[2]
            q = torch.empty(R, Hq * HD, device=x.device, dtype=x.dtype)
            if HD % 4 == 0:
                # q | k | v GEMM with RoPE and the cache write in its epilogue
                gemm_rope_packed(krms(x, b.n1), b.qkv.qp, b.qkv.sp, self.rope, pos, q, b.kc,
                                 b.vc, S, Hq, Hk, L, HD, b.qkv.K)
            else:
                qkv = gemm_packed(krms(x, b.n1), b.qkv.qp, b.qkv.sp, b.qkv.N, b.qkv.K)
                _rope_cache[(R, Hq + Hk)](qkv, self.rope, pos, q, b.kc, b.vc, S, Hq, Hk, L,
                                          HD=HD, HALF=next_power_of_2(HD // 2))
            if HD == 128 and Hq // Hk <= 4:
                # causal flash attention on MFMA: each K/V tile is read once per 64-row block
                o = prefill_attn(q, b.kc, b.vc, pos, S, Hq, Hk)
            else:
                # one split per row: a prompt row attends at most the prompt (no empty splits,
                # no combine pass); the rows themselves give the parallelism
                o = self._attention(b, q, pos, S, splits=1)
            x = gemm_packed(o, b.o.qp, b.o.sp, b.o.N, b.o.K, res=x)
            mm = gemm_silu_packed(krms(x, b.n2), b.w13.qp, b.w13.sp, b.w13.N // 2, b.w13.K)
            x = gemm_packed(mm, b.w2.qp, b.w2.sp, b.w2.N, b.w2.K, res=x)
        return krms(x, self.norm)

    def decode(self, x, pos, S, final_norm=True, o0=None):
        """Fast path for few rows (app/engine.py:180-211): x [R, D] with R = B*S (row r -> batch
        r // S), pos [R] absolute positions; row r attends [0, pos[r]].

        Per layer: rms+qkv+RoPE/KV write (one kernel), attention (+ split combine),
        O projection + residual, rms+w1|w3+SiLU*mul (one kernel), w2 + residual.
        ``final_norm=False`` returns the residual stream before the stack's last RMSNorm, for a
        consumer that fuses that norm into its own GEMV (the codebook heads).  ``o0``: layer 0's
        attention output, its q|k|v, RoPE and cache slot already done (by the depth decoder's
        sampler); the step then starts at layer 0's O projection."""
        if any(b.qkv.qp is None for b in self.blocks):
            h = self.decode_reference(x, pos, S)
            return h if final_norm else None
        R = x.shape[0]
        t = next((t for t in (self.tail, self.tail2) if t is not None and R == t["M"]), None)
        if self.use_tail and t is not None:
            x = self._decode_tail(x, pos, S, t, o0)
            return krms(x, self.norm) if final_norm else x
        for i, b in enumerate(self.blocks):
            Hq, Hk, HD, L = b.h, b.kvh, b.hd, b.kc.shape[2]
            if i == 0 and o0 is not None:
                o = o0
            else:
                q = torch.empty(R, Hq * HD, device=x.device, dtype=x.dtype)
                rms_qkv_rope(x, b.n1, b.qkv.qp, b.qkv.s8, self.rope, pos, q, b.kc, b.vc, S, Hq, Hk,
                             L, HD, stream=b.qkv.stream)
                o = self._attention(b, q, pos, S)
            x = b.o(o, res=x)
            mm = rms_w13_silu(x, b.n2, b.w13.qp, b.w13.sp, b.w13.N // 2, stream=b.w13.stream)
            x = b.w2(mm, res=x)
        return krms(x, self.norm) if final_norm else x

    def _decode_tail(self, x, pos, S, t, o0=None, head=None):
        """Layer 0's rms + q|k|v + RoPE + cache write and attention run first: one
        ecd_layer_head launch where the shapes allow attention in the launch, else on their
        own; then all layer tails as one ecd_layer_stack launch where supported, else one
        ecd_layer_tail launch per layer: the O projection, the MLP, the next layer's rms +
        q|k|v + RoPE + cache write and (where the shapes allow) that layer's attention, else
        attention (+ split combine) as its own launches.  Returns the last
        layer's output (a buffer of the stack, valid until the next decode call).  With several
        rows per cache (S > 1) the rows of a cache hold consecutive positions.  ``t``: the
        buffers for R rows.  ``head``: run the stack plan that ends in that codebook head and
        return its logits (None when the stack launch cannot run; nothing is launched then)."""
        q = t["q"]
        att = t["att"] and self.tail_attention

        def nxt_of(b):
            return dict(n1=b.n1, wq=b.qkv.qp, sq=b.qkv.s8, rope=self.rope, pos=pos, q=q, kc=b.kc,
                        vc=b.vc, S=S, Hq=b.h, Hk=b.kvh, L=b.kc.shape[2], HD=b.hd)

        b0 = self.blocks[0]
        L0, F = b0.kc.shape[2], b0.w2.K

        def stack_ok(o):
            return att and self.use_stack and t["plan"] is not None and layer_stack_supported(
                len(self.blocks), t["M"], self.dim, F, b0.h, b0.kvh, b0.hd, L0, b0.w13.stream,
                self.tail_kv_nt) \
                and not any(_overlap(v, u) for v in (x, o) for u in t["stack"].values())

        if head is not None and not stack_ok(o0 if o0 is not None else t["ob"][1]):
            return None
        if o0 is not None:
            o = o0
        elif att:
            o = layer_head(x, nxt_of(b0), t["ob"][1], b0.w2.K, t["sync"], t["err"], t["ws"],
                           stream=b0.qkv.stream, no_wait=self.tail_no_wait, kv_nt=self.tail_kv_nt)
        else:
            rms_qkv_rope(x, b0.n1, b0.qkv.qp, b0.qkv.s8, self.rope, pos, q, b0.kc, b0.vc, S, b0.h,
                         b0.kvh, b0.kc.shape[2], b0.hd, stream=b0.qkv.stream)
            o = self._attention(b0, q, pos, S)
        if stack_ok(o):
            nl = len(self.blocks)
            plan, y = t["hplans"][head] if head is not None else (t["plan"], None)
            return layer_stack(plan, nl, o, x, t["stack"]["xs"][nl - 1], self.rope, pos, q,
                               t["sync"], t["err"], t["ws"], S, b0.h, b0.kvh, L0, b0.hd, F,
                               stream=b0.w13.stream, no_wait=self.tail_no_wait,
                               kv_nt=self.tail_kv_nt, y=y)
        for i, b in enumerate(self.blocks):
            nb = self.blocks[i + 1] if i + 1 < len(self.blocks) else None
            nxt = None if nb is None else nxt_of(nb)
            o_next = t["ob"][i % 2] if (att and nb is not None) else None
            x = layer_tail(o, x, b.o.qp, b.o.s8, b.n2, b.w13.qp, b.w13.sp, b.w2.qp, b.w2.s8,
                           t["x1"], t["mm"], t["xb"][i % 2], t["sync"], t["err"], t["ws"],
                           nxt=nxt, o_next=o_next, stream=b.w13.stream,
                           no_wait=self.tail_no_wait, kv_nt=self.tail_kv_nt)
            if nb is not None:
                o = o_next if o_next is not None else self._attention(nb, q, pos, S)
        return x

    def _attention(self, b, q, pos, S, splits=None):
        """Decode attention of block b for the rows of q (row r over cache slots [0, pos[r]],
        app/kernels.py:110-167).  Caches of at most ATT_SHORT slots, and prompt passes
        (``splits=1``: the rows give the parallelism), run one split per (row, kv head) that
        writes o itself.  Longer caches run the split attention with its merge in the same
        launch (ecd_decode_attn_merged: attention_kb workgroups of 8 splits per pair, so that
        the grid covers the CUs whatever the row count), on the stack's workspace."""
        R = q.shape[0]
        Hq, Hk, HD, L = b.h, b.kvh, b.hd, b.kc.shape[2]
        o = torch.empty_like(q)
        st = stream_ptr(q.device)
        if splits == 1 or L <= ATT_SHORT:
            _ffi.call("ecd_decode_attn", q.data_ptr(), b.kc.data_ptr(), b.vc.data_ptr(),
                      pos.data_ptr(), o.data_ptr(), None, None, None, R, S, Hq, Hk, L, HD, 1,
                      1.0 / math.sqrt(HD), st)
            return o
        kb = attention_kb(R, Hk, L)
        if self.att_ws is None or self.att_ws.numel() < R * Hq * kb * (2 + HD) or \
                self.att_cnt.numel() < R * Hk:
            raise RuntimeError("Stack._attention: the attention workspace is smaller than the call")
        _ffi.call("ecd_decode_attn_merged", q.data_ptr(), b.kc.data_ptr(), b.vc.data_ptr(),
                  pos.data_ptr(), o.data_ptr(), self.att_ws.data_ptr(), self.att_cnt.data_ptr(),
                  R, S, Hq, Hk, L, HD, kb, 1.0 / math.sqrt(HD), st)
        return o

    def decode_reference(self, x, pos, S):
        """The reference's launch sequence (app/engine.py:180-211) through the drop-in kernel
        entry points of kernels.py (unpacked weights, one launch per reference kernel, the
        reference's attention grid and split count)."""
        R = x.shape[0]
        for b in self.blocks:
            Hq, Hk, HD, L = b.h, b.kvh, b.hd, b.kc.shape[2]
            qkv = int8_mm(krms(x, b.n1), b.qkv.q8, b.qkv.s8)
            q = torch.empty(R, Hq * HD, device=x.device, dtype=x.dtype)
            _rope_cache[(R, Hq + Hk)](qkv, self.rope, pos, q, b.kc, b.vc, S, Hq, Hk, L,
                                      HD=HD, HALF=next_power_of_2(HD // 2))
            ns = 1 if L <= ATT_SHORT else 16
            o = torch.empty_like(q)
            pm = torch.empty(R * Hq * ns, device=x.device) if ns > 1 else o
            pl = torch.empty_like(pm) if ns > 1 else o
            pa = torch.empty(R * Hq * ns, HD, device=x.device) if ns > 1 else o
            _attn[(R, Hk, ns)](q, b.kc, b.vc, pos, o, pm, pl, pa, S, Hq, Hk, L,
                               1.0 / math.sqrt(HD), HD=HD, HDP=next_power_of_2(HD), G=Hq // Hk,
                               BLK=64 if HD <= 128 else 16, NSPLIT=ns, num_warps=4)
            if ns > 1:
                _attn_combine[(R * Hq,)](pm, pl, pa, o, HD=HD, HDP=next_power_of_2(HD), NSPLIT=ns)
            x = int8_mm(o, b.o.q8, b.o.s8, x)
            a = int8_mm(krms(x, b.n2), b.w13.q8, b.w13.s8)
            Fd = a.shape[1] // 2
            mm = torch.empty(R, Fd, device=x.device, dtype=x.dtype)
            _silu_mul[(R, cdiv(Fd, 1024))](a, mm, Fd, BLOCK=1024)
            x = int8_mm(mm, b.w2.q8, b.w2.s8, x)
        return krms(x, self.norm)


# ---------------------------------------------------------------- weights
class _TensorSource:
    """Name -> tensor access over a safetensors file or an in-memory dict."""

    def __init__(self, weights, dev):
        self.meta = {}
        if isinstance(weights, (str, Path)):
            from safetensors import safe_open
            self._f = safe_open(str(weights), "pt", device=str(dev))
            self._keys = set(self._f.keys())
            self.meta = json.loads((self._f.metadata() or {}).get("lite", "{}"))
            self._get = self._f.get_tensor
        else:
            self._keys = set(weights.keys())
            self._get = lambda k: weights[k].to(dev)

    def __contains__(self, k):
        return k in self._keys

    def get(self, k):
        return self._get(k)


# ---------------------------------------------------------------- model
class HeartMuLaLite:
    """Backbone + depth decoder of HeartMuLa on the gfx950 decode kernels (app/engine.py:215-477).

    ``weights`` is a ``mula_int8.safetensors``-format file or a dict of tensors with the same
    names (``<name>.q8`` int8, ``<name>.s8`` bf16, norm ``.scale`` bf16)."""

    def __init__(self, weights, device="cuda", dtype=None, backbone=BACKBONE, decoder=DECODER):
        self.dev = torch.device(device)
        if self.dev.type != "cuda":
            raise RuntimeError("HeartMuLaLite (gfx950 path) needs a ROCm GPU device")
        if dtype is None:
            dtype = torch.float16
        if dtype != torch.float16:
            raise TypeError("the gfx950 decode kernels compute in float16 (app/engine.py:219-222)")
        self.dt = dtype
        self.fast = True
        f = _TensorSource(weights, self.dev)
        self.meta = f.meta

        def p(name, norm=False):
            if name in f:
                t = f.get(name).to(dtype)
                return t if norm else Linear(w=t)
            q8, s8 = f.get(name + ".q8"), f.get(name + ".s8")
            return Linear(q8=q8.contiguous(), s8=s8.to(dtype).contiguous())

        def emb(name):
            if name in f:
                return Emb(w=f.get(name).to(dtype))
            return Emb(q8=f.get(name + ".q8"), s8=f.get(name + ".s8").to(dtype))

        self.bb_cfg, self.dec_cfg = dict(backbone), dict(decoder)
        self.backbone = Stack(p, "backbone", backbone)
        self.decoder = Stack(p, "decoder", decoder)
        # the backbone (2.8 GB at the 3B shape) is streamed once per frame; the depth decoder is
        # re-read by 7 passes per frame, so its loads stay cacheable (256 MB Infinity Cache)
        for st, streamed in ((self.backbone, True), (self.decoder, False)):
            for b in st.blocks:
                b.qkv.pack(stream=streamed)
                b.o.pack(stream=streamed)
                b.w13.pack(interleave=True, stream=streamed)
                b.w2.pack(stream=streamed)
        self.text_emb = emb("text_embeddings.weight")
        self.audio_emb = emb("audio_embeddings.weight")
        self.uncond = f.get("unconditional_text_embedding.weight").to(dtype)
        self.projection = p("projection.weight")
        self.c0_head = p("codebook0_head.weight")
        self.audio_head = [p(f"audio_head.{i}") for i in range(N_CB - 1)]
        self.c0_head.pack(stream=True)
        for lin in [self.projection, *self.audio_head]:
            lin.pack()
        # When one depth-decoder pass (its layers and a codebook head) fits in the Infinity Cache
        # beside the per-token rows, the backbone's attention reads its cache slots nontemporal
        # at every length, so that the decoder stays resident across the backbone's layers from
        # one frame to the next (1024-wide decoder: +0.2% frames/s at KV 750, +2.6% at 4096).
        # The reference decoder (~340 MB per pass) does not fit, and there plain loads of short
        # splits are faster.
        lins = [lin for b in self.decoder.blocks for lin in (b.qkv, b.o, b.w13, b.w2)]
        lins.append(self.audio_head[0])
        if all(lin.qp is not None for lin in lins):
            self.backbone.tail_kv_nt = sum(lin.qp.numel() for lin in lins) <= DECODER_RESIDENT
        # codebook-0 head and the projection share their input (the backbone state): one GEMV
        # over [c0 head rows, zero rows up to a multiple of 64, projection rows] gives the
        # logits and the first decoder pass's projected backbone rows
        self._c0proj = None
        c0, pr = self.c0_head, self.projection
        if c0.qp is not None and pr.qp is not None and c0.K == pr.K:
            n0 = -(-c0.N // 64) * 64
            pad = n0 - c0.N
            self._c0proj = Linear(
                q8=torch.cat([c0.q8, c0.q8.new_zeros(pad, c0.K), pr.q8]).contiguous(),
                s8=torch.cat([c0.s8, c0.s8.new_zeros(pad), pr.s8]).contiguous()).pack(stream=True)
            self._c0proj.n0 = n0
        self.muq_b = f.get("muq_linear.bias").to(dtype)
        self.cb_off = torch.arange(N_CB, device=self.dev) * AUDIO_VOCAB
        self.graphs = {}
        self.N = self.B = None
        self._next_rows = self._xnext = self._next_qkv = self._onext = None
        self._hlog = None  # logits buffers of the heads that run inside the decoder's stack

    def _embed_audio(self, cb, tok):
        """Embedding of codebook ``cb`` for tokens tok [B, 1] -> [B, D] (app/engine.py:307-308)."""
        return self.audio_emb.gather(tok, cb, AUDIO_VOCAB)

    # -------------------------------------------------- one frame (backbone + 7 decoder passes)
    def _frame_fast(self, last_h, cfg, topk, temp, pos=None, forced=None, logits_out=None,
                    noise=None, normed=True):
        """app/engine.py:328-343.  Sampling is one fused kernel per codebook (CFG, temperature,
        top-k, Exponential race) writing straight into the [B, 8] token tensor; its draws are
        keyed by the seed and the frame position ``pos`` (int64 device tensor, first element).
        ``forced`` [B, 8] replaces the samples (teacher forcing), ``logits_out`` collects the
        8 logit tensors, ``noise`` [8, N, V] fixes the Exponential draws (tests).
        ``normed=False``: last_h is the backbone's residual stream before its final RMSNorm,
        which the first GEMV then applies itself."""
        B = self.B
        if forced is None:
            samples = torch.empty(B, N_CB, dtype=torch.long, device=self.dev)
            if pos is None:
                pos = self._pos_prompt
        else:
            samples = forced

        # sampled codebooks 1..6: the sampler also writes the next pass's input row (the
        # precomputed projection of the token's embedding) and, where the table exists, runs
        # that pass's layer 0 up to its attention output (precomputed q|k|v of the token)
        nxt = self._next_rows if forced is None else None
        nqkv = self._next_qkv if nxt is not None else None
        d0 = self.decoder.blocks[0] if nqkv is not None else None

        def pick(i, lg, rows=None, qkv=None, x=None, ev=None, xe=None):
            if logits_out is not None:
                logits_out.append(lg)
            if forced is None:
                att = {} if qkv is None else dict(qkv=qkv, kc=d0.kc, vc=d0.vc, p=i + 1,
                                                  o=self._onext)
                if rows is not None and x is None:
                    x = self._xnext
                sample_topk(lg, self.N, cfg, temp, topk, samples[:, i], seed=self._seed, pos=pos,
                            salt=i, noise=None if noise is None else noise[i], rows=rows,
                            x=x, ev=ev, xe=xe, **att)
            return samples[:, i:i + 1]

        # decoder pass 0: two rows per batch entry (backbone state, codebook-0 embedding)
        cp = self._c0proj if nxt is not None else None
        if cp is None and not normed:
            last_h = krms(last_h, self.backbone.norm)
        if cp is not None:
            # one GEMV for the codebook-0 logits and the projected backbone rows (with the
            # backbone's final RMSNorm as its prologue when last_h is not normed yet); the
            # sampler puts those (even rows) and its token's precomputed row (odd rows) into _x0
            y = torch.empty(B, cp.N, device=self.dev, dtype=torch.float16)
            if normed:
                gemv_packed(last_h, cp.qp, cp.s8, cp.N, cp.K, out=y, stream=True)
            else:
                rms_gemv_packed(last_h, self.backbone.norm, cp.qp, cp.s8, cp.N, cp.K,
                                stream=True, out=y)
            pick(0, y[:, :AUDIO_VOCAB], nxt[0], x=self._x0[1::2], ev=y[:, cp.n0:],
                 xe=self._x0[0::2])
            lg = self._decode_head0(self._x0)
        else:
            c0 = pick(0, self._c0(last_h))
            lg = self._decode_head0(self._project(c0, 0, even=last_h))
        for i in range(1, N_CB):
            rows = nxt[i] if nxt is not None and i < N_CB - 1 else None
            qkv = nqkv[i - 1] if rows is not None and nqkv is not None else None
            ci = pick(i, lg, rows, qkv)
            if i < N_CB - 1:
                x = self._xnext if rows is not None else self._project(ci, i)
                lg = self._decode_head(x, self._pass_pos[i - 1], i,
                                       o0=None if qkv is None else self._onext)
        return samples

    def _packed_decoder(self):
        return self.audio_head[0].qp is not None and bool(self.decoder.blocks) and \
            self.decoder.blocks[0].qkv.qp is not None

    def _decode(self, x, pos, S, o0=None):
        """Decoder pass; with packed heads the stack's final RMSNorm is left to the head GEMV.
        ``o0``: layer 0's attention output when the sampler ran layer 0 up to it."""
        if self._packed_decoder():
            return self.decoder.decode(x, pos, S, final_norm=False, o0=o0)
        return self.decoder.decode(x, pos, S, o0=o0)

    def _decode_head0(self, x):
        """The first decoder pass (two rows per take) and audio_head[0] of its odd rows: one
        layer-stack launch that ends in the head (on all rows) where its plan exists, else the
        pass and the head GEMV on the odd rows."""
        lg = None
        if self._hlog is not None:
            lg = self.decoder.decode_head(x, self._pass0_pos, 2, 0)
        if lg is not None:
            return lg[1::2]
        return self._head(0, self._decode(x, self._pass0_pos, 2)[1::2])

    def _decode_head(self, x, pos, i, o0=None):
        """Decoder pass i (1 .. 6, one row per take) and audio_head[i] of its output: one
        layer-stack launch that ends in the head where its plan exists, else the pass and the
        head GEMV."""
        lg = None
        if self._hlog is not None:
            lg = self.decoder.decode_head(x, pos, 1, i, o0=o0)
        return lg if lg is not None else self._head(i, self._decode(x, pos, 1, o0=o0))

    def _logits(self, M, N):
        """[M, N] fp16 logits whose rows start 128-byte aligned (the sampler loads 16 B/lane)."""
        return torch.empty(M, -(-N // 64) * 64, device=self.dev, dtype=torch.float16)[:, :N]

    def _c0(self, h):
        """codebook0_head(h) into aligned logit rows."""
        hd = self.c0_head
        if hd.qp is not None and hd.sp is hd.s8:
            return gemv_packed(h, hd.qp, hd.s8, hd.N, hd.K, out=self._logits(h.shape[0], hd.N),
                               stream=hd.stream)
        return hd(h)

    def _head(self, i, h):
        """audio_head[i](decoder.norm(h)) -- norm fused into the head GEMV when packed."""
        hd = self.audio_head[i]
        if hd.qp is not None and self.decoder.blocks and self.decoder.blocks[0].qkv.qp is not None:
            return rms_gemv_packed(h, self.decoder.norm, hd.qp, hd.s8, hd.N, hd.K,
                                   stream=hd.stream, out=self._logits(h.shape[0], hd.N))
        return hd(h)

    def _project(self, tok, cb, even=None):
        """projection(_embed_audio(cb, tok)) -- with ``even`` the interleave (even[b], emb[b]) --
        as one GEMV whose prologue gathers the int8 embedding rows (app/engine.py:336-342)."""
        pr, e = self.projection, self.audio_emb
        if pr.qp is None:
            x = e.gather(tok, cb, AUDIO_VOCAB, even=even)
            return pr(x)
        ev = None if even is None else even.contiguous()
        return embed_gemv_packed(tok, e.table, e.scales, cb, AUDIO_VOCAB, pr.qp, pr.s8, pr.N, even=ev)

    def _step(self, tok, pos, bucket, cfg, topk, temp, **kw):
        """tok [B, 8] previous frame; pos [B, 1] (app/engine.py:345-349).  Where the frame's
        first GEMV takes the backbone's final RMSNorm as its prologue, the backbone step returns
        its residual stream."""
        h = self.audio_emb.sum_codebooks(tok, AUDIO_VOCAB)
        fused = kw.get("forced") is None and self._next_rows is not None and \
            self._c0proj is not None and all(b.qkv.qp is not None for b in self.backbone.blocks)
        hb = self.backbone.decode(h, pos[:, 0].contiguous(), 1, final_norm=not fused)
        return self._frame_fast(hb, cfg, topk, temp, pos=pos, normed=not fused, **kw)

    # -------------------------------------------------- caches
    def alloc(self, n, L, cfg_scale=1.5, seed=None):
        """Static caches for n takes and backbone capacity L (app/engine.py:380-388), and the
        sampler's seed (drawn from torch's host generator when not given)."""
        self.N = n
        self.B = 2 * n if cfg_scale != 1.0 else n
        if seed is None or seed < 0:
            seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        self._seed = torch.tensor([seed], dtype=torch.int64, device=self.dev)
        self._pos_prompt = torch.zeros(1, dtype=torch.int64, device=self.dev)
        # depth-decoder slots: pass 0 runs the row pairs (backbone state, codebook-0 token) at
        # slots 0 and 1 of each take's cache; pass i = 1 .. 6 writes slot i + 1
        self._pass0_pos = torch.arange(2 * self.B, device=self.dev) % 2
        self._pass_pos = torch.arange(2, N_CB, device=self.dev).repeat_interleave(self.B) \
            .view(N_CB - 2, self.B)
        self.backbone.alloc(self.B, L, self.dev, self.dt)
        self.decoder.alloc(self.B, N_CB, self.dev, self.dt)
        # passes 1 .. 6 end in their codebook head inside the decoder's stack launch where the
        # stack supports it: one logits buffer per head
        self._hlog = None
        if self._packed_decoder():
            # (the first pass's head runs on its 2B rows; the odd ones are the codebook-1 logits)
            self._hlog = {i: self._logits(self.B, AUDIO_VOCAB) for i in range(1, N_CB - 1)}
            self._hlog[0] = self._logits(2 * self.B, AUDIO_VOCAB)
            self.decoder.head_plans({i: (self.audio_head[i], y) for i, y in self._hlog.items()})
        self._alloc_next_rows()

    @torch.no_grad()
    def _alloc_next_rows(self):
        """The decoder input of passes 1..6 is projection(_embed_audio(i, ci)) (app/engine.py:343),
        a function of (codebook, token) and the weights only: rows[i][t] holds it for every
        token t of codebooks i = 0..6 (weight preprocessing, like the packing), and the frame's
        sampler copies the sampled token's row into the [B, D] buffer ``_xnext`` (codebook 0:
        the odd rows of the first pass's [2B, D] input ``_x0``).  Each row comes from the
        frame's own projection kernel with its numerics (one launch per codebook over all V
        tokens; the rows of a launch do not interact), so it is bit-equal to the per-frame
        projection it replaces.  Kept across allocations with the same B."""
        pr, e = self.projection, self.audio_emb
        B = self.B
        if pr.qp is None or self.dt != torch.float16:
            self._next_rows = self._xnext = self._next_qkv = self._onext = None
            return
        if getattr(self, "_next_rows", None) is not None and self._xnext.shape[0] == B:
            return
        self._next_rows = self._xnext = self._next_qkv = self._onext = None
        V = AUDIO_VOCAB
        rows = torch.empty(N_CB - 1, V, pr.N, device=self.dev, dtype=torch.float16)
        tok = torch.arange(V, device=self.dev).view(-1, 1)
        for cb in range(N_CB - 1):
            # all V tokens in one launch, with the per-row numerics of the frame's B-row launch
            embed_gemv_packed(tok, e.table, e.scales, cb, V, pr.qp, pr.s8, pr.N, out=rows[cb],
                              dense=False)
        self._next_rows = rows
        self._xnext = torch.empty(B, pr.N, device=self.dev, dtype=torch.float16)
        self._x0 = torch.empty(2 * B, pr.N, device=self.dev, dtype=torch.float16)
        self._alloc_next_qkv()

    @torch.no_grad()
    def _alloc_next_qkv(self):
        """Layer 0 of decoder pass i (1..6) starts with rms -> q|k|v -> RoPE at position i + 1
        (app/engine.py:189-199) on the input row of the sampled token: again a function of
        (codebook, token) and the weights.  qkv[i - 1][t] holds q heads | k heads | v heads of
        token t (the per-op kernel rms_qkv_rope writing whole rows, one launch per codebook,
        with the per-row numerics of a decode step), so the sampler can write the cache slot and
        run that layer's attention itself; only for the head_dims (128, 384) and the pair
        counts the sampler's folded attention takes."""
        self._next_qkv = self._onext = None
        d0 = self.decoder.blocks[0] if self.decoder.blocks else None
        B, V = self.B, AUDIO_VOCAB
        if d0 is None or d0.qkv.qp is None or d0.hd not in (128, 384) or d0.h % d0.kvh or \
                d0.h // d0.kvh > 4:
            return
        pairs, slots = (4, 16) if d0.hd == 128 else (8, 8)
        if (2 if B == 2 * self.N else 1) * d0.kvh > pairs or N_CB - 1 >= slots:
            return
        Hq, Hk, HD, L = d0.h, d0.kvh, d0.hd, d0.kc.shape[2]
        if L < N_CB:
            return
        qkv = torch.empty(N_CB - 2, V, (Hq + 2 * Hk) * HD, device=self.dev, dtype=torch.float16)
        for cb in range(1, N_CB - 1):
            # every token of codebook cb in one launch, its q | k | v row written in place
            pos = torch.full((V,), cb + 1, dtype=torch.int64, device=self.dev)
            rms_qkv_rope_rows(self._next_rows[cb], d0.n1, d0.qkv.qp, d0.qkv.s8, self.decoder.rope,
                              pos, qkv[cb - 1], Hq, Hk, HD, dense=False)
        self._next_qkv = qkv
        self._onext = torch.empty(B, Hq * HD, device=self.dev, dtype=torch.float16)

    # -------------------------------------------------- generation
    @torch.inference_mode()
    def generate(self, text, muq_idx, *, max_ms=60_000, temperature=1.0, topk=50, cfg_scale=1.5,
                 seed=None, use_graphs=True, progress=None, abort=None, n=1, forced=None):
        """A song of up to ``max_ms`` for n takes (app/engine.py:374-448) with the prompt given as
        token ids ``text`` [P] (int64) and the muq slot index.  Returns [8, T] if n == 1, else a
        list of n such tensors, each take cut before its first frame holding an EOS token.
        ``forced`` [max_ms // 80 + 1, B, 8] int64 on the device replaces the sampled tokens of
        every frame (teacher forcing a whole song).  Every 25 frames (and at the end) the host
        reads the takes' EOS frames together with the layer tails' error words, and raises
        RuntimeError if a tail launch timed out at a gate."""
        if seed is not None and seed >= 0:
            torch.manual_seed(seed)
        text = torch.as_tensor(text, dtype=torch.int64)
        P = int(text.numel())
        n_frames = max_ms // FRAME_MS
        cap = P + n_frames + 2 + 256
        self.alloc(n, cap, cfg_scale)
        N, B = self.N, self.B
        if forced is not None and tuple(forced.shape) != (n_frames + 1, B, N_CB):
            raise ValueError(f"generate: forced must be [{n_frames + 1}, {B}, {N_CB}]")

        # prompt pass (text rows, the muq slot's bias, unconditional rows for CFG)
        h = self.text_emb(text.to(self.dev)).unsqueeze(0).repeat(B, 1, 1)
        h[:N, muq_idx] = self.muq_b
        if B == 2 * N:
            h[N:] = self.uncond[0]
        hb = self.backbone(h, torch.arange(P, device=self.dev).unsqueeze(0).expand(B, P), P, None)

        # song state on the device: next input tokens and position, the frames so far, and
        # each take's first EOS frame (-1 while it runs)
        st = dict(tok=torch.empty(B, N_CB, dtype=torch.long, device=self.dev),
                  pos=torch.full((B, 1), P - 1, dtype=torch.long, device=self.dev),
                  out=torch.empty(n_frames + 1, N, N_CB, dtype=torch.long, device=self.dev),
                  eos=torch.full((N,), -1, dtype=torch.long, device=self.dev),
                  forced=None if forced is None else forced[0].clone())
        kw = {} if forced is None else {"forced": st["forced"]}
        first = self._frame_fast(hb[:, -1].contiguous(), cfg_scale, topk, temperature,
                                 pos=st["pos"], **kw)
        self._advance(first, st, P, n_frames)

        key = (B, cap, topk, float(temperature), float(cfg_scale))
        done = n_frames
        ends = None
        for i in range(n_frames):
            if abort and abort():
                self.release()
                return None
            if forced is not None:
                st["forced"].copy_(forced[i + 1])
            if use_graphs:
                g = self.graphs.get(key)
                if g is None:
                    g = self.graphs[key] = self._capture(st, cap, cfg_scale, topk, temperature,
                                                         song=(P, n_frames))
                g[0].replay()
            else:
                self._advance(self._step(st["tok"], st["pos"], cap, cfg_scale, topk, temperature,
                                         **kw), st, P, n_frames)
            if (i + 1) % 25 == 0 or i == n_frames - 1:
                ends = self._song_status(st["eos"])
                if min(ends) >= 0:
                    done = i + 1
                    break
                if progress:
                    progress((i + 1) * FRAME_MS / 1000, max_ms / 1000)
        if ends is None:
            ends = self._song_status(st["eos"])
        self.frames_run = done
        res = [st["out"][: (e if e >= 0 else done + 1), c].t().clone() for c, e in enumerate(ends)]
        self.release()
        return res[0] if n == 1 else res

    def _song_status(self, eos):
        """Each take's first EOS frame (-1 while it runs) and the layer tails' error words, in
        one device -> host read (the song loop's only one).  A set error word means a gate wait
        of a persistent tail launch gave up (a workgroup of its grid was not resident, e.g.
        another process held CUs): the frames since the last read are undefined, so the gate
        state is cleared, the caches are released and the song stops with RuntimeError."""
        errs = [s.tail["err"] for s in (self.backbone, self.decoder) if s.tail is not None]
        vals = torch.cat([eos, *[e.to(eos.dtype) for e in errs]]).tolist()
        n = eos.numel()
        if any(vals[n:]):
            failed = [nm for nm, v in zip(("backbone", "decoder"), vals[n:]) if v]
            self.tail_reset()
            self.release()
            raise RuntimeError(f"layer-tail launch of the {' and '.join(failed)} timed out at a "
                               "gate (its grid was not all resident); the song was stopped")
        return vals[:n]

    def tail_error(self):
        """True if a layer-tail launch of either stack timed out since the last reset."""
        return self.backbone.tail_error() or self.decoder.tail_error()

    def tail_reset(self):
        """Zero both stacks' gate regions, workspaces and error words (their contents are
        undefined after a timeout)."""
        self.backbone.tail_reset()
        self.decoder.tail_reset()

    def _advance(self, samples, st, P, n_frames):
        """Frame bookkeeping on the device: samples -> next input, frame stored, first EOS frame
        per take recorded, position + 1 (one kernel, capturable)."""
        _ffi.call("ecd_frame_advance", samples.data_ptr(), samples.stride(0), st["tok"].data_ptr(),
                  st["tok"].stride(0), st["pos"].data_ptr(), st["pos"].stride(0),
                  st["out"].data_ptr(), st["eos"].data_ptr(), self.B, self.N, P, n_frames,
                  AUDIO_EOS, stream_ptr(self.dev))

    def _capture(self, static, bucket, cfg, topk, temp, song=None):
        """One eager warm-up, then ``_step`` captured into a hipGraph (app/engine.py:450-461).
        With ``song`` = (P, n_frames) the graph ends with the frame bookkeeping (``_advance``),
        so consecutive replays make consecutive frames with no host work in between."""
        kw = {"forced": static["forced"]} if static.get("forced") is not None else {}
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self._step(static["tok"], static["pos"], bucket, cfg, topk, temp, **kw)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        # a layer-tail wait that gave up in this warm-up (seen on a persistent kernel's first
        # dispatch on a stream): its outputs are discarded and the replays redo its cache
        # writes, so the gate regions are cleared; a timeout in a replay still raises (the song
        # loop reads the error words)
        if self.tail_error():
            warnings.warn("a layer-tail wait of the capture's eager warm-up gave up (error words "
                          f"backbone {self.backbone.tail_error():#x}, decoder "
                          f"{self.decoder.tail_error():#x}); gate regions cleared", RuntimeWarning)
            self.tail_reset()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=getattr(self, "_pool", None)):
            out = self._step(static["tok"], static["pos"], bucket, cfg, topk, temp, **kw)
            if song is not None:
                self._advance(out, static, *song)
        self._pool = g.pool()
        return g, out

    def release(self):
        self.graphs.clear()
        self._pool = None
        self.backbone.free()
        self.decoder.free()
        torch.cuda.empty_cache()

    def vram_weights(self):
        """Device bytes of the model's weights: every distinct tensor behind the linear layers
        (int8 codes, scales, packed tile copies, interleaved scales), the embedding tables,
        norm vectors and biases, and the per-token tables built at alloc."""
        seen, total = set(), 0
        lins = [getattr(b, n) for st in (self.backbone, self.decoder) for b in st.blocks
                for n in ("qkv", "o", "w13", "w2")]
        lins += [self.projection, self.c0_head, *self.audio_head]
        if self._c0proj is not None:
            lins.append(self._c0proj)
        ts = [t for lin in lins for t in (lin.q8, lin.s8, lin.qp, lin.sp)]
        ts += [t for e in (self.text_emb, self.audio_emb) for t in (e.w, e.q8, e.s8)]
        ts += [t for st in (self.backbone, self.decoder) for b in st.blocks for t in (b.n1, b.n2)]
        ts += [self.backbone.norm, self.decoder.norm, self.uncond, self.muq_b, self._next_rows,
               self._next_qkv]
        for t in ts:
            if t is not None and t.data_ptr() not in seen:
                seen.add(t.data_ptr())
                total += t.numel() * t.element_size()
        return total
