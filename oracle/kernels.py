"""Kernel-level oracle of the decode path (test infrastructure only).

Each function restates one reference kernel with its fp16 rounding points; sums are
evaluated in float64 (any summation order of the reference's fp32 accumulators lies
within the fp16 output tolerance of this value).
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import f16, f32, hadd, hmul
from .rope import apply_rope


# ---------------------------------------------------------------- int8 GEMV
def gemv_i8(x, q, s, res=None) -> np.ndarray:
    """int8_mm (app/kernels.py:40-54).

    M <= 16 rows (_gemv8, :20-37):  y = fp16(fp32(acc) * fp32(s)), acc = sum_k x * q (fp32)
    M  > 16 rows (dense, :46-49):   y = fp16(x @ fp16(fp16(q) * s).T)
    then y = fp16(y + res)."""
    x = np.asarray(x, dtype=np.float16)
    shp = x.shape
    x2 = x.reshape(-1, shp[-1]).astype(np.float64)
    q = np.asarray(q, dtype=np.int8)
    s = np.asarray(s, dtype=np.float16)
    M = x2.shape[0]
    if M > 16:
        y = f16(_dot_rows_f64(x2, q, s).astype(np.float32))
    else:
        acc = _dot_rows_f64(x2, q).astype(np.float32)
        y = f16(acc * s.astype(np.float32)[None, :])
    if res is not None:
        y = hadd(y, np.asarray(res, dtype=np.float16).reshape(M, -1))
    return y.reshape(*shp[:-1], q.shape[0])


_F64_BUF = [np.empty(0)]
# Accumulation type of the GEMV sums.  float64 is the oracle; tests switch it to float32 (the
# blocked fp32 sums of a BLAS GEMM, another valid summation order) to measure how far a model
# output moves under fp32 re-association alone -- the noise floor of a deep composite.
GEMV_ACC = [np.float64]


def _dot_rows_f64(x2, q, s=None) -> np.ndarray:
    """x2 [M, K] @ w[N, K]^T summed in GEMV_ACC (float64) with w = q, or with ``s`` the
    dequantised w = fp16(fp16(q) * s) of the dense path.  w is formed in row chunks inside one
    reused buffer (large weights: no per-call float64 copy of the whole matrix)."""
    acc = GEMV_ACC[0]
    N, Kd = q.shape
    rows = N if N * Kd <= (1 << 22) else max(1, (1 << 22) // Kd)
    if _F64_BUF[0].size < rows * Kd:
        _F64_BUF[0] = np.empty(rows * Kd, np.float64)
    x2 = x2.astype(acc, copy=False)
    out = np.empty((x2.shape[0], N), acc)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        b = _F64_BUF[0][: (r1 - r0) * Kd].view(acc)[: (r1 - r0) * Kd].reshape(r1 - r0, Kd)
        if s is None:
            np.copyto(b, q[r0:r1], casting="unsafe")
        else:
            np.copyto(b, hmul(q[r0:r1].astype(np.float16), s[r0:r1, None]), casting="unsafe")
        out[:, r0:r1] = x2 @ b.T
    return out


# ---------------------------------------------------------------- RMSNorm
def rms(x, w, eps=1e-5) -> np.ndarray:
    """_rms (app/kernels.py:58-67): fp16(fp16(x * inv) * w), inv = 1/sqrt(sum(x^2)/D + eps)."""
    xf = np.asarray(x, dtype=np.float16).astype(np.float32)
    D = xf.shape[-1]
    ss = (xf.astype(np.float64) ** 2).sum(-1, keepdims=True)
    inv = (1.0 / np.sqrt(ss / D + np.float64(np.float32(eps)))).astype(np.float32)
    return hmul(f16(xf * inv), np.asarray(w, dtype=np.float16))


# ---------------------------------------------------------------- RoPE + cache write
def rope_kv_write(qkv, rope, pos, kc, vc, S, Hq, Hk, HD) -> np.ndarray:
    """_rope_cache (app/kernels.py:78-107).  Writes kc/vc in place at [r // S, kh, pos[r]];
    returns the rotated q [R, Hq * HD]."""
    qkv = np.asarray(qkv, dtype=np.float16)
    R = qkv.shape[0]
    pos = np.asarray(pos, dtype=np.int64)
    cs = np.asarray(rope, dtype=np.float32)[pos]                       # [R, HD/2, 2]
    qh = qkv[:, : Hq * HD].reshape(R, Hq, HD)
    kh = qkv[:, Hq * HD: (Hq + Hk) * HD].reshape(R, Hk, HD)
    vh = qkv[:, (Hq + Hk) * HD:].reshape(R, Hk, HD)
    q = apply_rope(qh, cs[:, None])
    k = apply_rope(kh, cs[:, None])
    for r in range(R):
        b = r // S
        kc[b, :, pos[r]] = k[r]
        vc[b, :, pos[r]] = vh[r]
    return q.reshape(R, Hq * HD)


# ---------------------------------------------------------------- decode attention
def decode_attn(q, kc, vc, pos, S, Hq, Hk, HD, scale=None, nsplit=16, blk=None):
    """Flash-decoding GQA attention, the reference tiling (app/kernels.py:111-153).

    Row r attends slots [0, pos[r]] of kv head kh with query heads kh*G .. kh*G+G-1.
    The range is cut into nsplit chunks of ceil(ceil(len/nsplit)/blk)*blk tokens; each
    chunk runs an online softmax over blk-token tiles: scores fp32 (q.k) * scale, running
    max, exp, probabilities rounded to fp16 for the P.V product, fp32 running sum.
    Returns the split partials (m, l, acc) with shapes [R, Hq, nsplit], [R, Hq, nsplit],
    [R, Hq, nsplit, HD]."""
    G = Hq // Hk
    if scale is None:
        scale = 1.0 / math.sqrt(HD)
    if blk is None:
        blk = 64 if HD <= 128 else 16
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    R = q.shape[0]
    q = q.reshape(R, Hq, HD)
    pos = np.asarray(pos, dtype=np.int64)
    L = kc.shape[2]
    pm = np.full((R, Hq, nsplit), -np.inf, np.float32)
    pl = np.zeros((R, Hq, nsplit), np.float32)
    pa = np.zeros((R, Hq, nsplit, HD), np.float32)
    sc32 = np.float32(scale)
    for r in range(R):
        b = r // S
        ln = int(min(max(pos[r] + 1, 0), L))
        chunk = -(-(-(-ln // nsplit)) // blk) * blk
        for kh in range(Hk):
            K = kc[b, kh].astype(np.float64)
            V = vc[b, kh].astype(np.float64)
            qg = q[r, kh * G:(kh + 1) * G]                               # [G, HD]
            for sp in range(nsplit):
                lo, hi = sp * chunk, min(ln, sp * chunk + chunk)
                m = np.full(G, -np.inf, np.float32)
                l = np.zeros(G, np.float32)
                acc = np.zeros((G, HD), np.float64)
                for s0 in range(lo, hi, blk):
                    s1 = min(s0 + blk, hi)
                    sc = (qg @ K[s0:s1].T).astype(np.float32) * sc32      # [G, t]
                    m_new = np.maximum(m, sc.max(1))
                    alpha = np.exp((m - m_new).astype(np.float64)).astype(np.float32)
                    pe = np.exp((sc - m_new[:, None]).astype(np.float64)).astype(np.float32)
                    l = (l * alpha + pe.sum(1, dtype=np.float64)).astype(np.float32)
                    pv = f16(pe).astype(np.float64) @ V[s0:s1]
                    acc = acc * alpha[:, None] + pv
                    m = m_new
                pm[r, kh * G:(kh + 1) * G, sp] = m
                pl[r, kh * G:(kh + 1) * G, sp] = l
                pa[r, kh * G:(kh + 1) * G, sp] = acc
    return pm, pl, pa


def attn_combine(pm, pl, pa) -> np.ndarray:
    """_attn_combine (app/kernels.py:156-167): LSE merge over the split axis, empty splits
    (m = -inf) weighted 0.  pm/pl [..., NS], pa [..., NS, HD] -> fp16 [..., HD]."""
    M = pm.max(-1, keepdims=True)
    w = np.where(pm > -np.inf, np.exp((pm - M).astype(np.float64)), 0.0)
    num = (pa.astype(np.float64) * w[..., None]).sum(-2)
    den = (pl.astype(np.float64) * w).sum(-1)
    return f16((num / den[..., None]).astype(np.float32))


def decode_attn_out(q, kc, vc, pos, S, Hq, Hk, HD, nsplit=16, blk=None) -> np.ndarray:
    """Flash-decoding attention followed by the combine: o [R, Hq * HD] fp16."""
    pm, pl, pa = decode_attn(q, kc, vc, pos, S, Hq, Hk, HD, nsplit=nsplit, blk=blk)
    o = attn_combine(pm, pl, pa)
    return o.reshape(o.shape[0], Hq * HD)


def attention_exact(q, kc, vc, pos, S, Hq, Hk, HD) -> np.ndarray:
    """Textbook softmax(q K^T / sqrt(HD)) V over [0, pos] in float64 -- the closed form the
    flash-decoding restatement must agree with (no fp16 rounding of probabilities)."""
    G = Hq // Hk
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    R = q.shape[0]
    q = q.reshape(R, Hq, HD)
    out = np.zeros((R, Hq, HD), np.float64)
    for r in range(R):
        b = r // S
        ln = int(pos[r]) + 1
        for h in range(Hq):
            kh = h // G
            K = kc[b, kh, :ln].astype(np.float64)
            V = vc[b, kh, :ln].astype(np.float64)
            sc = K @ q[r, h] / math.sqrt(HD)
            p = np.exp(sc - sc.max())
            out[r, h] = p @ V / p.sum()
    return out.reshape(R, Hq * HD)


# ---------------------------------------------------------------- SiLU(a) * b
def silu_mul(x) -> np.ndarray:
    """_silu_mul (app/kernels.py:171-180): fp16(fp16(a / (1 + exp(-a))) * b) with a = x[:, :F],
    b = x[:, F:], silu evaluated in fp32."""
    x = np.asarray(x, dtype=np.float16)
    F = x.shape[-1] // 2
    a = x[..., :F].astype(np.float32)
    with np.errstate(over="ignore"):
        sg = f16(a / (np.float32(1.0) + np.exp(-a)))
    return hmul(sg, x[..., F:])


# ---------------------------------------------------------------- int8 embeddings
def embed_rows(q8, s16, rows) -> np.ndarray:
    """Emb.__call__ (app/engine.py:95-98): fp16(q8[rows]) * s16[rows] in fp16."""
    rows = np.asarray(rows, dtype=np.int64)
    return hmul(np.asarray(q8)[rows].astype(np.float16), np.asarray(s16)[rows][..., None])


def embed_sum(q8, s16, tok, vocab) -> np.ndarray:
    """Backbone input (app/engine.py:348): audio_emb(tok + cb_off).sum(1, dtype=fp16) --
    fp32 accumulation over the codebooks, one fp16 rounding."""
    tok = np.asarray(tok, dtype=np.int64)
    C = tok.shape[1]
    rows = tok + np.arange(C, dtype=np.int64)[None, :] * vocab
    return sum_rows(embed_rows(q8, s16, rows))


def sum_rows(e) -> np.ndarray:
    """[B, C, D] fp16 -> fp16(sum over C in fp32) (the .sum(1, dtype=fp16) of app/engine.py:348)."""
    e = np.asarray(e, np.float16).astype(np.float32)
    acc = np.zeros((e.shape[0], e.shape[2]), np.float32)
    for c in range(e.shape[1]):
        acc = (acc + e[:, c]).astype(np.float32)
    return f16(acc)
