"""Decode-path kernels with the entry points of the reference's ``app/kernels.py``.

Same names, argument order and tensor layouts as the reference, so an engine written
against it runs unchanged:

    int8_mm(x, w, s, res=None)                                   app/kernels.py:40-54
    rms(x, w, eps=1e-5)                                          app/kernels.py:70-74
    _rope_cache[grid](qkv, rope, pos, q, kc, vc, S, Hq, Hk, L, HD=, HALF=)    :78-107
    _attn[grid](q, kc, vc, pos, o, pm, pl, pa, S, Hq, Hk, L, scale,
                HD=, HDP=, G=, BLK=, NSPLIT=, num_warps=)                     :111-153
    _attn_combine[grid](pm, pl, pa, o, HD=, HDP=, NSPLIT=)                    :156-167
    _silu_mul[grid](x, y, F_, BLOCK=)                                         :171-180

Every call goes to a hand-written gfx950 HIP kernel through the C ABI of
``libecdecode.so``, on the current HIP stream, so it can be captured in a hipGraph.
The Triton tiling knobs (HALF, HDP, BLK, BLOCK, num_warps) are accepted for drop-in
compatibility and checked for consistency, but the HIP kernels choose their own tiling;
the grid must be the one the reference launches with.  Tensors must be fp16 (the
reference GPU default, app/engine.py:219-222) and live on a ROCm device.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _ffi

__all__ = ["int8_mm", "rms", "_rope_cache", "_attn", "_attn_combine", "_silu_mul",
           "next_power_of_2", "cdiv", "stream_ptr"]


def next_power_of_2(n: int) -> int:
    """Host helper the reference engine takes from Triton (app/engine.py:192,194)."""
    n = int(n)
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def cdiv(a: int, b: int) -> int:
    return -(-int(a) // int(b))


def stream_ptr(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _dev(t: torch.Tensor, name: str) -> torch.device:
    if not t.is_cuda:
        raise RuntimeError(f"{name}: the decode path runs only on a ROCm GPU tensor (got {t.device})")
    return t.device


def _f16(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.float16:
        raise TypeError(f"{name}: expected float16, got {t.dtype}")


def _ptr(t):
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------- GEMV int8 (+ optional residual)
def int8_mm(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, res: torch.Tensor | None = None):
    """x [..., K] fp16, w [N, K] int8, s [N] fp16 -> [..., N] (+ res).

    M = prod(x.shape[:-1]) <= 16 uses the reference GEMV numerics (scale after the fp32
    dot product); M > 16 uses its dequantise-then-GEMM numerics (app/kernels.py:46-49)."""
    dev = _dev(x, "int8_mm")
    _f16(x, "int8_mm x")
    if w.dtype != torch.int8 or w.dim() != 2 or not w.is_contiguous():
        raise TypeError("int8_mm: w must be a contiguous [N, K] int8 tensor")
    if s.dtype != torch.float16 or s.numel() != w.shape[0] or not s.is_contiguous():
        raise TypeError("int8_mm: s must be a contiguous [N] float16 tensor")
    shp = x.shape
    K = shp[-1]
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"int8_mm: x has K={K}, w has K={w.shape[1]}")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) < K:
        x2 = x2.contiguous()
    M = x2.shape[0]
    y = torch.empty(M, N, device=dev, dtype=torch.float16)
    r2 = None
    if res is not None:
        _f16(res, "int8_mm res")
        r2 = res.reshape(M, N)
        if r2.stride(-1) != 1 or r2.stride(0) < N:
            r2 = r2.contiguous()
    if M == 0:
        return y.reshape(*shp[:-1], N)
    _ffi.call("ecd_gemv_i8", x2.data_ptr(), x2.stride(0), w.data_ptr(), s.data_ptr(), _ptr(r2),
              r2.stride(0) if r2 is not None else 0, y.data_ptr(), N, M, N, K, int(M > 16),
              stream_ptr(dev))
    return y.reshape(*shp[:-1], N)


# ---------------------------------------------------------------- RMSNorm
def rms(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5):
    """x [R, D] fp16, w [D] fp16 -> fp16(fp16(x * rsqrt(mean(x^2) + eps)) * w)."""
    dev = _dev(x, "rms")
    _f16(x, "rms x")
    _f16(w, "rms w")
    R, D = x.shape
    if w.numel() != D:
        raise ValueError("rms: weight size mismatch")
    if x.stride(-1) != 1:
        x = x.contiguous()
    y = torch.empty(R, D, device=dev, dtype=torch.float16)
    _ffi.call("ecd_rmsnorm", x.data_ptr(), x.stride(0), w.data_ptr(), y.data_ptr(), D, R, D,
              float(eps), stream_ptr(dev))
    return y


class _Launcher:
    """``kernel[grid](...)`` call syntax of the reference's Triton launchers."""

    def __init__(self, name, fn, grid_fn):
        self.__name__ = name
        self._fn = fn
        self._grid_fn = grid_fn

    def __getitem__(self, grid):
        grid = tuple(grid) if isinstance(grid, (tuple, list)) else (grid,)

        def launch(*args, **kwargs):
            want = self._grid_fn(*args, **kwargs)
            if tuple(grid) != tuple(want):
                raise ValueError(f"{self.__name__}: grid {grid} does not match the launch {want}")
            return self._fn(*args, **kwargs)

        return launch

    def __call__(self, *args, **kwargs):  # direct call without a grid
        return self._fn(*args, **kwargs)


# ---------------------------------------------------------------- RoPE + KV-cache write
def _rope_cache_impl(qkv, rope, pos, q, kc, vc, S, Hq, Hk, L, HD, HALF=None):
    dev = _dev(qkv, "_rope_cache")
    for t, n in ((qkv, "qkv"), (q, "q"), (kc, "kc"), (vc, "vc")):
        _f16(t, f"_rope_cache {n}")
        if not t.is_contiguous():
            raise ValueError(f"_rope_cache: {n} must be contiguous")
    if rope.dtype != torch.float32 or not rope.is_contiguous():
        raise TypeError("_rope_cache: rope table must be contiguous float32 [L, HD/2, 2]")
    if pos.dtype != torch.int64 or not pos.is_contiguous():
        raise TypeError("_rope_cache: pos must be contiguous int64")
    if HALF is not None and HALF < HD // 2:
        raise ValueError("_rope_cache: HALF must cover HD // 2")
    R = qkv.shape[0]
    if qkv.shape[1] != (Hq + 2 * Hk) * HD or q.numel() != R * Hq * HD or pos.numel() != R:
        raise ValueError("_rope_cache: shape mismatch")
    if kc.shape[-1] != HD or kc.shape[-2] != L or kc.shape[1] != Hk or kc.shape[0] * S < R:
        raise ValueError("_rope_cache: cache must be [B, Hk, L, HD] with B >= R / S")
    if rope.shape[0] < L or rope.shape[1] != HD // 2:
        raise ValueError("_rope_cache: rope table must have >= L rows of HD/2 pairs")
    _ffi.call("ecd_rope_kv_write", qkv.data_ptr(), rope.data_ptr(), pos.data_ptr(), q.data_ptr(),
              kc.data_ptr(), vc.data_ptr(), R, S, Hq, Hk, L, HD, stream_ptr(dev))


_rope_cache = _Launcher("_rope_cache", _rope_cache_impl,
                        lambda qkv, rope, pos, q, kc, vc, S, Hq, Hk, L, HD=None, HALF=None:
                        (qkv.shape[0], Hq + Hk))


# ---------------------------------------------------------------- decode attention
def _attn_impl(q, kc, vc, pos, o, pm, pl, pa, S, Hq, Hk, L, scale, HD, HDP=None, G=None,
               BLK=None, NSPLIT=16, num_warps=None):
    dev = _dev(q, "_attn")
    for t, n in ((q, "q"), (kc, "kc"), (vc, "vc"), (o, "o")):
        _f16(t, f"_attn {n}")
        if not t.is_contiguous():
            raise ValueError(f"_attn: {n} must be contiguous")
    if pos.dtype != torch.int64 or not pos.is_contiguous():
        raise TypeError("_attn: pos must be contiguous int64")
    if G is not None and G != Hq // Hk:
        raise ValueError("_attn: G must equal Hq // Hk")
    R = q.shape[0]
    if q.numel() != R * Hq * HD or pos.numel() != R or o.numel() != R * Hq * HD:
        raise ValueError("_attn: shape mismatch")
    if kc.shape[-1] != HD or kc.shape[-2] != L or kc.shape[1] != Hk or kc.shape[0] * S < R:
        raise ValueError("_attn: cache must be [B, Hk, L, HD] with B >= R / S")
    if NSPLIT > 1:
        need = R * Hq * NSPLIT
        for t, n, k in ((pm, "pm", need), (pl, "pl", need), (pa, "pa", need * HD)):
            if t.dtype != torch.float32 or t.numel() < k or not t.is_contiguous():
                raise ValueError(f"_attn: {n} must be float32 with >= {k} elements")
        ptrs = (pm.data_ptr(), pl.data_ptr(), pa.data_ptr())
    else:
        ptrs = (None, None, None)
    _ffi.call("ecd_decode_attn", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
              o.data_ptr(), *ptrs, R, S, Hq, Hk, L, HD, int(NSPLIT), float(scale), stream_ptr(dev))


_attn = _Launcher("_attn", _attn_impl,
                  lambda q, kc, vc, pos, o, pm, pl, pa, S, Hq, Hk, L, scale, HD=None, HDP=None,
                  G=None, BLK=None, NSPLIT=16, num_warps=None: (q.shape[0], Hk, NSPLIT))


def _attn_combine_impl(pm, pl, pa, o, HD, HDP=None, NSPLIT=16):
    dev = _dev(o, "_attn_combine")
    _f16(o, "_attn_combine o")
    RH = o.numel() // HD
    for t, n, k in ((pm, "pm", RH * NSPLIT), (pl, "pl", RH * NSPLIT), (pa, "pa", RH * NSPLIT * HD)):
        if t.dtype != torch.float32 or t.numel() < k or not t.is_contiguous():
            raise ValueError(f"_attn_combine: {n} must be float32 with >= {k} elements")
    _ffi.call("ecd_attn_combine", pm.data_ptr(), pl.data_ptr(), pa.data_ptr(), o.data_ptr(), RH,
              HD, int(NSPLIT), stream_ptr(dev))


_attn_combine = _Launcher("_attn_combine", _attn_combine_impl,
                          lambda pm, pl, pa, o, HD=None, HDP=None, NSPLIT=16: (o.numel() // HD,))


def decode_attn_noalloc(q, kc, vc, pos, S, Hq, Hk, L, scale, nsplit=16, out=None):
    """_attn + _attn_combine in one call whose split partials live in the library's static
    device workspace (8 MiB per GPU): nothing is allocated when ``out`` is given, so it can run
    under hipGraph capture without a memory pool.  Raises MemoryError when R * Hq * nsplit
    partials do not fit.  Calls overlapping on one GPU share the workspace."""
    dev = _dev(q, "decode_attn_noalloc")
    for t, n in ((q, "q"), (kc, "kc"), (vc, "vc")):
        _f16(t, f"decode_attn_noalloc {n}")
        if not t.is_contiguous():
            raise ValueError(f"decode_attn_noalloc: {n} must be contiguous")
    if pos.dtype != torch.int64 or not pos.is_contiguous():
        raise TypeError("decode_attn_noalloc: pos must be contiguous int64")
    R = q.shape[0]
    HD = kc.shape[-1]
    if q.numel() != R * Hq * HD or pos.numel() != R or kc.shape[1] != Hk or kc.shape[-2] != L \
            or kc.shape[0] * S < R or vc.shape != kc.shape:
        raise ValueError("decode_attn_noalloc: shape mismatch")
    o = out if out is not None else torch.empty_like(q)
    if o.shape != q.shape or o.dtype != torch.float16 or not o.is_contiguous():
        raise ValueError("decode_attn_noalloc: out must be a contiguous fp16 tensor shaped like q")
    _ffi.call("ecd_decode_attn_noalloc", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
              o.data_ptr(), R, S, Hq, Hk, L, HD, int(nsplit), float(scale), stream_ptr(dev))
    return o


# ---------------------------------------------------------------- SiLU(a) * b
def _silu_mul_impl(x, y, F_, BLOCK=None):
    dev = _dev(x, "_silu_mul")
    _f16(x, "_silu_mul x")
    _f16(y, "_silu_mul y")
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("_silu_mul: tensors must be contiguous")
    R = y.numel() // F_
    if x.numel() != 2 * R * F_:
        raise ValueError("_silu_mul: x must be [R, 2F] for y [R, F]")
    _ffi.call("ecd_silu_mul", x.data_ptr(), y.data_ptr(), R, F_, stream_ptr(dev))


_silu_mul = _Launcher("_silu_mul", _silu_mul_impl,
                      lambda x, y, F_, BLOCK=1024: (y.numel() // F_, cdiv(F_, BLOCK)))


# ---------------------------------------------------------------- fused sampler
def sample_topk(logits, N, cfg, temp, topk, out, seed=None, pos=None, salt=0, noise=None,
                rows=None, x=None, qkv=None, kc=None, vc=None, p=0, o=None, ev=None, xe=None):
    """CFG mix + temperature + top-k + softmax(log_softmax) + Exponential race in one kernel
    (the math of _sample/_guided, app/engine.py:291-305).

    logits [B, V] fp16 (B = 2N: cond rows then uncond rows; B = N: no CFG); out: int64 view
    with out[b] the token slot of row b (any row stride).  The Exponential(1) draws come from
    a counter-based Philox keyed by seed (int64 device scalar) at frame position pos (int64
    device scalar) and ``salt``, or from ``noise`` [N, V] float32 when given.

    With ``rows`` [>= V, D] fp16 and ``x`` [B, D] fp16, row b of x also receives rows[token of
    row b] (zeros where the race had no winner): the next decoder pass's input when rows[t]
    holds projection(embedding of token t) (app/engine.py:343).  With ``qkv`` [>= V,
    (Hq + 2 Hk) * HD] fp16 as well (the next pass's layer-0 q | k | v of each token at slot
    ``p``), k and v also go to slot p of the caches ``kc`` / ``vc`` [B, Hk, L, HD] and each
    row's decode attention over slots 0 .. p goes to ``o`` [B, Hq * HD] (HD = 128, or 384 with
    the arithmetic of the short-cache attention kernel).  With ``ev`` and ``xe`` ([>= B, D]
    each), rows of ev are copied to the same rows of xe as they are."""
    dev = _dev(logits, "sample_topk")
    _f16(logits, "sample_topk logits")
    B, V = logits.shape
    if logits.stride(-1) != 1:
        raise ValueError("sample_topk: logits rows must be contiguous")
    if out.dtype != torch.int64 or out.shape[0] != B:
        raise ValueError("sample_topk: out must be int64 with one slot per row")
    if noise is not None:
        if noise.dtype != torch.float32 or tuple(noise.shape) != (N, V) or not noise.is_contiguous():
            raise ValueError("sample_topk: noise must be contiguous float32 [N, V]")
    elif seed is None or pos is None:
        raise ValueError("sample_topk: seed and pos device scalars are required without noise")
    if (rows is None) != (x is None):
        raise ValueError("sample_topk: rows and x go together")
    if rows is None:
        _ffi.call("ecd_sample_topk", logits.data_ptr(), logits.stride(0), B, N, float(cfg),
                  float(temp), int(topk), V, _ptr(noise), _ptr(seed), _ptr(pos), int(salt),
                  out.data_ptr(), out.stride(0), stream_ptr(dev))
        return
    _f16(rows, "sample_topk rows")
    _f16(x, "sample_topk x")
    D = x.shape[1]
    if rows.dim() != 2 or rows.shape[0] < V or rows.shape[1] != D or rows.stride(1) != 1 or \
            x.dim() != 2 or x.shape[0] < B or x.stride(1) != 1:
        raise ValueError("sample_topk: rows must be [>= V, D] and x [>= B, D] with contiguous rows")
    Hq = Hk = L = HD = 0
    if qkv is not None:
        _f16(qkv, "sample_topk qkv")
        _f16(o, "sample_topk o")
        _f16(kc, "sample_topk kc")
        _f16(vc, "sample_topk vc")
        if kc.dim() != 4:
            raise ValueError("sample_topk: caches must be [>= B, Hk, L, HD]")
        Hk, L, HD = kc.shape[1], kc.shape[2], kc.shape[3]
        Hq = o.shape[1] // HD
        if HD not in (128, 384) or kc.shape[0] < B or vc.shape != kc.shape or \
                not kc.is_contiguous() or not vc.is_contiguous() or o.shape[0] < B or \
                o.stride(1) != 1 or qkv.dim() != 2 or qkv.shape[1] != (Hq + 2 * Hk) * HD or \
                qkv.stride(1) != 1:
            raise ValueError("sample_topk: qkv [>= V, (Hq + 2 Hk) HD], caches [>= B, Hk, L, HD], "
                             "o [>= B, Hq HD], HD 128 or 384")
    if (ev is None) != (xe is None):
        raise ValueError("sample_topk: ev and xe go together")
    if ev is not None:
        _f16(ev, "sample_topk ev")
        _f16(xe, "sample_topk xe")
        if ev.shape[0] < B or xe.shape[0] < B or ev.shape[1] != D or xe.shape[1] != D or \
                ev.stride(1) != 1 or xe.stride(1) != 1:
            raise ValueError("sample_topk: ev and xe must be [>= B, D] with contiguous rows")
    _ffi.call("ecd_sample_topk_next", logits.data_ptr(), logits.stride(0), B, N, float(cfg),
              float(temp), int(topk), V, _ptr(noise), _ptr(seed), _ptr(pos), int(salt),
              out.data_ptr(), out.stride(0), rows.data_ptr(), rows.stride(0), rows.shape[0],
              x.data_ptr(), x.stride(0), D, _ptr(qkv), 0 if qkv is None else qkv.stride(0),
              0 if qkv is None else qkv.shape[0], _ptr(kc), _ptr(vc), L, int(p), _ptr(o),
              0 if o is None else o.stride(0), Hq, Hk, HD, _ptr(ev),
              0 if ev is None else ev.stride(0),
              _ptr(xe), 0 if xe is None else xe.stride(0), stream_ptr(dev))


# ---------------------------------------------------------------- packed weights + fused GEMVs
def pack_i8(w: torch.Tensor, interleave: bool = False) -> torch.Tensor:
    """Lane-ordered 16 x 64 tile layout of an int8 [N, K] matrix (K % 64 == 0) for the fused
    GEMVs.  With ``interleave`` the two halves of w are row-interleaved (w1 | w3 -> pairs)."""
    dev = _dev(w, "pack_i8")
    if w.dtype != torch.int8 or w.dim() != 2 or not w.is_contiguous():
        raise TypeError("pack_i8: w must be a contiguous [N, K] int8 tensor")
    N, K = w.shape
    if K % 64 or (interleave and N % 2):
        raise ValueError("pack_i8: K must be a multiple of 64 (and N even to interleave)")
    out = torch.empty(-(-N // 16) * 16 * K, dtype=torch.int8, device=dev)
    _ffi.call("ecd_pack_i8", w.data_ptr(), N, K, int(interleave), out.data_ptr(), stream_ptr(dev))
    return out


def _check_x(x, K, name):
    _dev(x, name)
    _f16(x, name + " x")
    if x.dim() != 2 or x.shape[1] != K or x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        raise ValueError(f"{name}: x must be [M, {K}] fp16 with unit inner stride, 16-byte rows")


def _flags(M, stream):
    return int(M > 16) | (2 if stream else 0)


def gemv_packed(x, wp, s, N, K, res=None, out=None, stream=False):
    """y = int8_mm(x, w, s, res) on packed weights (same numerics).  ``stream``: the weights are
    read once per frame (nontemporal loads)."""
    _check_x(x, K, "gemv_packed")
    M = x.shape[0]
    y = out if out is not None else torch.empty(M, N, device=x.device, dtype=torch.float16)
    if res is not None:
        _f16(res, "gemv_packed res")
        if res.shape != (M, N) or res.stride(1) != 1:
            raise ValueError("gemv_packed: res must be [M, N] with unit inner stride")
    _ffi.call("ecd_gemv_i8p", x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(), _ptr(res),
              res.stride(0) if res is not None else 0, y.data_ptr(), y.stride(0), M, N, K,
              _flags(M, stream), 0, 0, stream_ptr(x.device))
    return y


def gemv_packed_splitk(x, wp, s, N, K, ks, res=None, stream=False):
    """gemv_packed with K split over ``ks`` workgroups per tile (fp32 partial sums added in a
    fixed order by a second kernel): for few output tiles over a long K, where one workgroup
    per tile leaves most CUs idle.  Same numerics up to the fp32 summation order."""
    _check_x(x, K, "gemv_packed_splitk")
    M = x.shape[0]
    y = torch.empty(M, N, device=x.device, dtype=torch.float16)
    ws = torch.empty(ks * M * N, device=x.device, dtype=torch.float32)
    if res is not None:
        _f16(res, "gemv_packed_splitk res")
        if res.shape != (M, N) or res.stride(1) != 1:
            raise ValueError("gemv_packed_splitk: res must be [M, N] with unit inner stride")
    _ffi.call("ecd_gemv_i8p_splitk", x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(),
              _ptr(res), res.stride(0) if res is not None else 0, y.data_ptr(), y.stride(0), M, N,
              K, int(ks), ws.data_ptr(), _flags(M, stream), stream_ptr(x.device))
    return y


def gemm_packed(x, wp, s, N, K, res=None):
    """int8_mm(x, w, s, res) for many rows (the dense numerics, y = fp16(x @ fp16(q * s)^T))
    on packed weights, tiled on MFMA; ``res`` is added in fp16."""
    _check_x(x, K, "gemm_packed")
    M = x.shape[0]
    y = torch.empty(M, N, device=x.device, dtype=torch.float16)
    if res is not None:
        _f16(res, "gemm_packed res")
        if res.shape != (M, N) or res.stride(1) != 1:
            raise ValueError("gemm_packed: res must be [M, N] with unit inner stride")
    _ffi.call("ecd_gemm_i8p", x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(), _ptr(res),
              res.stride(0) if res is not None else 0, y.data_ptr(), y.stride(0), M, N, K,
              stream_ptr(x.device))
    return y


def gemm_silu_packed(x, wp, s, F, K):
    """_silu_mul(int8_mm(x, w1|w3, s)) for many rows on row-interleaved packed w1|w3
    (pack_i8(..., interleave=True)) -> [M, F]."""
    _check_x(x, K, "gemm_silu_packed")
    M = x.shape[0]
    mm = torch.empty(M, F, device=x.device, dtype=torch.float16)
    _ffi.call("ecd_gemm_i8p_silu", x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(),
              mm.data_ptr(), mm.stride(0), M, F, K, stream_ptr(x.device))
    return mm


def gemm_rope_packed(x, wp, s, rope, pos, q, kc, vc, S, Hq, Hk, L, HD, K):
    """int8_mm(x, wq|wk|wv, s) followed by _rope_cache (app/kernels.py:78-107) in one launch:
    the q | k | v GEMM of many rows with RoPE and the cache write in its epilogue.  pos [M] int64
    (row m -> batch item m // S); writes q [M, Hq * HD] and the cache slots of kc / vc."""
    _check_x(x, K, "gemm_rope_packed")
    M = x.shape[0]
    for t, nm in ((q, "q"), (kc, "kc"), (vc, "vc")):
        _f16(t, f"gemm_rope_packed {nm}")
        if not t.is_contiguous():
            raise ValueError(f"gemm_rope_packed: {nm} must be contiguous")
    if q.shape != (M, Hq * HD):
        raise ValueError("gemm_rope_packed: q must be [M, Hq * HD]")
    if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
        raise ValueError("gemm_rope_packed: pos must be a contiguous int64 vector of M rows")
    if rope.dtype != torch.float32 or not rope.is_contiguous() or rope.numel() < L * HD:
        raise ValueError("gemm_rope_packed: rope must be a contiguous fp32 [L, HD] table")
    if kc.shape[1:] != (Hk, L, HD) or vc.shape != kc.shape or kc.shape[0] * S < M:
        raise ValueError("gemm_rope_packed: kc / vc must be [B, Hk, L, HD] with B * S >= M")
    _ffi.call("ecd_gemm_i8p_rope", x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(),
              rope.data_ptr(), pos.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), M, S,
              Hq, Hk, L, HD, K, stream_ptr(x.device))
    return q


def pack_f16(w: torch.Tensor, interleave: bool = False) -> torch.Tensor:
    """Lane-ordered 16 x 64 tile layout (2 KB tiles) of an fp16 [N, K] matrix (K % 64 == 0) for
    the fp16-weight GEMM; ``interleave`` row-interleaves the two halves (gate | up -> pairs)."""
    dev = _dev(w, "pack_f16")
    if w.dtype != torch.float16 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("pack_f16: w must be a contiguous fp16 [N, K] matrix")
    N, K = w.shape
    out = torch.empty(_ffi.lib().ecd_packed_bytes_f16(N, K) // 2, device=dev, dtype=torch.float16)
    _ffi.call("ecd_pack_f16", w.data_ptr(), N, K, int(interleave), out.data_ptr(), stream_ptr(dev))
    return out


def gemm_f16_packed(x, wp, N, K, bias=None, alpha=1.0, res=None, out=None):
    """F.linear(x, w, bias) on packed fp16 weights (fp32 accumulation and bias, one fp16 rounding),
    optionally scaled by ``alpha`` (rounded again) and plus ``res`` (fp16 add) -> [M, N]."""
    _check_x(x, K, "gemm_f16_packed")
    M = x.shape[0]
    y = out if out is not None else torch.empty(M, N, device=x.device, dtype=torch.float16)
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N):
        raise ValueError("gemm_f16_packed: bias must be fp32 [N]")
    _ffi.call("ecd_gemm_f16p", x.data_ptr(), x.stride(0), wp.data_ptr(),
              bias.data_ptr() if bias is not None else None, float(alpha),
              res.data_ptr() if res is not None else None, res.stride(0) if res is not None else 0,
              y.data_ptr(), y.stride(0), M, N, K, stream_ptr(x.device))
    return y


def gemm_f16_silu_packed(x, wp, F, K, out=None):
    """silu(x @ gate^T) * (x @ up^T) on interleaved packed fp16 gate | up -> [M, F]."""
    _check_x(x, K, "gemm_f16_silu_packed")
    M = x.shape[0]
    mm = out if out is not None else torch.empty(M, F, device=x.device, dtype=torch.float16)
    if mm.shape != (M, F) or mm.dtype != torch.float16 or mm.stride(1) != 1:
        raise ValueError("gemm_f16_silu_packed: out must be fp16 [M, F] with unit inner stride")
    _ffi.call("ecd_gemm_f16p_silu", x.data_ptr(), x.stride(0), wp.data_ptr(), mm.data_ptr(),
              mm.stride(0), M, F, K, stream_ptr(x.device))
    return mm


def prefill_attn(q, kc, vc, pos, S, Hq, Hk, scale=None, out=None):
    """Causal prompt-pass attention on MFMA: q [B*S, Hq*HD] fp16, kc/vc [B, Hk, L, HD] holding
    the prompt's K/V, pos [B*S] int64 -> o [B*S, Hq*HD] (row r attends slots [0, pos[r]])."""
    R = q.shape[0]
    B, _, L, HD = kc.shape
    if q.dtype != torch.float16 or not q.is_contiguous() or q.shape[1] != Hq * HD or R != B * S:
        raise ValueError("prefill_attn: q must be contiguous fp16 [B*S, Hq*HD]")
    if not (kc.is_contiguous() and vc.is_contiguous()) or pos.dtype != torch.int64:
        raise ValueError("prefill_attn: contiguous caches and int64 positions required")
    o = out if out is not None else torch.empty_like(q)
    if o.shape != q.shape or o.dtype != torch.float16 or not o.is_contiguous():
        raise ValueError("prefill_attn: out must be a contiguous fp16 tensor shaped like q")
    pc = pos.contiguous()
    _ffi.call("ecd_prefill_attn", q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
              pc.data_ptr(), o.data_ptr(), B, S, Hq, Hk, L, HD,
              float(scale if scale is not None else 1.0 / math.sqrt(HD)), stream_ptr(q.device))
    return o


def rms_gemv_packed(x, nw, wp, s, N, K, eps=1e-5, stream=False, out=None):
    """int8_mm(rms(x, nw), w, s) in one kernel.  ``out``: optional [M, N] fp16 destination with
    unit inner stride (any row stride)."""
    _check_x(x, K, "rms_gemv_packed")
    M = x.shape[0]
    y = out if out is not None else torch.empty(M, N, device=x.device, dtype=torch.float16)
    if y.shape != (M, N) or y.dtype != torch.float16 or y.stride(1) != 1:
        raise ValueError("rms_gemv_packed: out must be fp16 [M, N] with unit inner stride")
    _ffi.call("ecd_rms_gemv_i8p", x.data_ptr(), x.stride(0), nw.data_ptr(), float(eps), wp.data_ptr(),
              s.data_ptr(), y.data_ptr(), y.stride(0), M, N, K, _flags(M, stream), stream_ptr(x.device))
    return y


def rms_qkv_rope(x, nw, wp, s, rope, pos, q, kc, vc, S, Hq, Hk, L, HD, eps=1e-5, stream=False):
    """rms -> fused q|k|v GEMV -> RoPE of q and k -> q out, k/v into the cache at pos (one kernel)."""
    K = x.shape[1]
    _check_x(x, K, "rms_qkv_rope")
    M = x.shape[0]
    if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
        raise ValueError("rms_qkv_rope: pos must be contiguous int64 [M]")
    if kc.shape != (kc.shape[0], Hk, L, HD) or kc.shape[0] * S < M or vc.shape != kc.shape:
        raise ValueError("rms_qkv_rope: caches must be [B, Hk, L, HD] with B * S >= M")
    if rope.shape[0] < L or rope.shape[1] != HD // 2 or rope.dtype != torch.float32:
        raise ValueError("rms_qkv_rope: rope table must be float32 [>= L, HD/2, 2]")
    if q.numel() != M * Hq * HD or not (q.is_contiguous() and kc.is_contiguous() and vc.is_contiguous()):
        raise ValueError("rms_qkv_rope: q/kc/vc must be contiguous")
    _ffi.call("ecd_rms_qkv_rope", x.data_ptr(), x.stride(0), nw.data_ptr(), float(eps), wp.data_ptr(),
              s.data_ptr(), rope.data_ptr(), pos.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
              M, S, Hq, Hk, L, HD, K, _flags(M, stream), stream_ptr(x.device))


def rms_qkv_rope_rows(x, nw, wp, s, rope, pos, out, Hq, Hk, HD, eps=1e-5, dense=False):
    """rms -> fused q|k|v GEMV -> RoPE of q and k at pos[m] -> out[m] = q | k | v of row m
    ([M, (Hq + 2Hk) HD], row stride N, no cache write), one kernel for any M.  ``dense=False``
    keeps the numerics of a decode step of at most 16 rows (per-row scale after the int8 sum)
    whatever M is."""
    K = x.shape[1]
    _check_x(x, K, "rms_qkv_rope_rows")
    M = x.shape[0]
    N = (Hq + 2 * Hk) * HD
    if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
        raise ValueError("rms_qkv_rope_rows: pos must be contiguous int64 [M]")
    if rope.dim() != 3 or rope.shape[1] != HD // 2 or rope.dtype != torch.float32:
        raise ValueError("rms_qkv_rope_rows: rope table must be float32 [L, HD/2, 2]")
    _f16(out, "rms_qkv_rope_rows out")
    if out.shape != (M, N) or not out.is_contiguous() or out.data_ptr() % 16:
        raise ValueError(f"rms_qkv_rope_rows: out must be contiguous [{M}, {N}]")
    L = rope.shape[0]
    _ffi.call("ecd_rms_qkv_rope", x.data_ptr(), x.stride(0), nw.data_ptr(), float(eps), wp.data_ptr(),
              s.data_ptr(), rope.data_ptr(), pos.data_ptr(), out.data_ptr(), None, None,
              M, 1, Hq, Hk, L, HD, K, int(bool(dense)) | 4, stream_ptr(x.device))
    return out


def rms_w13_silu(x, nw, wp, s_il, F, eps=1e-5, stream=False):
    """rms -> [w1 | w3] GEMV on row-interleaved packed weights -> fp16(silu(a)) * b, [M, F]."""
    K = x.shape[1]
    _check_x(x, K, "rms_w13_silu")
    M = x.shape[0]
    mm = torch.empty(M, F, device=x.device, dtype=torch.float16)
    _ffi.call("ecd_rms_w13_silu", x.data_ptr(), x.stride(0), nw.data_ptr(), float(eps), wp.data_ptr(),
              s_il.data_ptr(), mm.data_ptr(), M, F, K, _flags(M, stream), stream_ptr(x.device))
    return mm


def layer_tail_supported(M, D, F, Hq, Hk, HD, L=1, attention=False):
    """True when ``layer_tail`` runs these shapes on the current device (with ``attention``: the
    next layer's attention over an L-slot cache inside the same launch)."""
    return _ffi.lib().ecd_layer_tail_supported(int(M), int(D), int(F), int(Hq), int(Hk), int(HD),
                                               int(L), int(bool(attention))) == _ffi.ECD_OK


def layer_tail_ws_bytes(D, Hq, Hk, HD):
    """Bytes of the layer-tail workspace for these shapes on the current device."""
    return int(_ffi.lib().ecd_layer_tail_ws_bytes(int(D), int(Hq), int(Hk), int(HD)))


def layer_tail(o, xin, wo, so, n2, w13, s13, w2, s2, x1, mm, xout, sync, err, ws, nxt=None,
               o_next=None, eps=1e-5, stream=False, no_wait=False, kv_nt=False):
    """One launch for the tail of a decode layer (app/engine.py:206-210: O projection +
    residual, rms -> w1|w3 -> SiLU * mul, w2 + residual) and, with ``nxt``, the next layer's
    rms -> q|k|v -> RoPE -> q, cache slot (:189-192) and, with ``o_next`` [M, Hq * HD], that
    layer's decode attention (:194-204) into o_next.  Writes x1 [M, D], mm [M, F] and the layer
    output xout [M, D] (which must not alias xin, o, x1 or mm).  ``nxt``: dict with n1, wq
    (packed), sq, rope, pos, q, kc, vc, S, Hq, Hk, L, HD.  ``sync`` (int32 [>= 4096], zero before
    first use) and ``err`` (int32 [1]) persist between calls; ``ws``: float32 workspace of
    layer_tail_ws_bytes bytes, zero before first use and kept with its ``sync`` (partials are
    recognised by the sync region's gate count).  ``no_wait``: every wait gives up at once (tests
    of the error path: err becomes 1 and sync, ws and err must be zeroed before the next call).
    ``kv_nt``: the attention reads every cache slot with nontemporal loads (else only splits of
    more than 32 slots), for callers whose other data should stay in the Infinity Cache."""
    dev = _dev(o, "layer_tail")
    M, D = o.shape
    F = mm.shape[1]
    for t, n in ((o, "o"), (xin, "xin"), (x1, "x1"), (mm, "mm"), (xout, "xout")):
        _f16(t, f"layer_tail {n}")
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise ValueError(f"layer_tail: {n} must be contiguous and 16-byte aligned")
    if xin.shape != (M, D) or x1.shape != (M, D) or xout.shape != (M, D) or mm.shape[0] != M:
        raise ValueError("layer_tail: o, xin, x1, xout must be [M, D] and mm [M, F]")
    lo, hi = xout.data_ptr(), xout.data_ptr() + xout.numel() * 2
    for t in (o, xin, x1, mm):
        if t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * 2:
            raise ValueError("layer_tail: xout must not alias o, xin, x1 or mm")
    if sync.dtype != torch.int32 or sync.numel() < 4096 or sync.data_ptr() % 256:
        raise ValueError("layer_tail: sync must be int32 [>= 4096], 256-byte aligned")
    if err.dtype != torch.int32 or err.numel() < 1:
        raise ValueError("layer_tail: err must be int32 [1]")
    if ws.dtype != torch.float32 or ws.data_ptr() % 16:
        raise ValueError("layer_tail: ws must be float32, 16-byte aligned")
    if nxt is None:
        nargs = [None] * 8
        S = Hq = Hk = L = HD = 1
    else:
        n = nxt
        pos, kc = n["pos"], n["kc"]
        S, Hq, Hk, L, HD = n["S"], n["Hq"], n["Hk"], n["L"], n["HD"]
        if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
            raise ValueError("layer_tail: pos must be contiguous int64 [M]")
        if kc.shape != (kc.shape[0], Hk, L, HD) or kc.shape[0] * S < M or n["vc"].shape != kc.shape:
            raise ValueError("layer_tail: caches must be [B, Hk, L, HD] with B * S >= M")
        if n["q"].numel() != M * Hq * HD or not n["q"].is_contiguous():
            raise ValueError("layer_tail: q must be contiguous [M, Hq * HD]")
        if n["rope"].shape[0] < L or n["rope"].shape[1] != HD // 2:
            raise ValueError("layer_tail: rope table must be float32 [>= L, HD/2, 2]")
        nargs = [n["n1"].data_ptr(), n["wq"].data_ptr(), n["sq"].data_ptr(), n["rope"].data_ptr(),
                 pos.data_ptr(), n["q"].data_ptr(), kc.data_ptr(), n["vc"].data_ptr()]
    if ws.numel() * 4 < layer_tail_ws_bytes(D, Hq, Hk, HD):
        raise ValueError("layer_tail: ws is smaller than layer_tail_ws_bytes")
    if o_next is not None:
        if nxt is None:
            raise ValueError("layer_tail: o_next needs the next layer (nxt)")
        _f16(o_next, "layer_tail o_next")
        if o_next.numel() != M * Hq * HD or not o_next.is_contiguous() or o_next.data_ptr() % 16:
            raise ValueError("layer_tail: o_next must be contiguous [M, Hq * HD]")
    _ffi.call("ecd_layer_tail", o.data_ptr(), xin.data_ptr(), wo.data_ptr(), so.data_ptr(),
              n2.data_ptr(), w13.data_ptr(), s13.data_ptr(), w2.data_ptr(), s2.data_ptr(), *nargs,
              _ptr(o_next), x1.data_ptr(), mm.data_ptr(), xout.data_ptr(), sync.data_ptr(),
              err.data_ptr(),
              ws.data_ptr(), M, D, F, S, Hq, Hk, L, HD, float(eps),
              _flags(M, stream) | (4 if no_wait else 0) | (8 if kv_nt else 0), stream_ptr(dev))
    return xout


# order of a layer record of ecd_layer_stack (ecd_layer_rec)
STACK_FIELDS = ("wo", "so", "n2", "w13", "s13", "w2", "s2", "n1", "wq", "sq", "kc", "vc", "x1",
                "mm", "xout", "o_next", "y")


def layer_stack_supported(nl, M, D, F, Hq, Hk, HD, L, stream=False, kv_nt=False):
    """True when ``layer_stack`` runs nl layers of these shapes with these weight / cache-load
    modes."""
    return _ffi.lib().ecd_layer_stack_supported(
        int(nl), int(M), int(D), int(F), int(Hq), int(Hk), int(HD), int(L),
        (2 if stream else 0) | (8 if kv_nt else 0)) == _ffi.ECD_OK


def layer_stack_layers_per_launch(nl, M, D, F, Hq, Hk, HD, L, stream=False, kv_nt=False):
    """Layers per kernel launch of a ``layer_stack`` call (0 when not supported)."""
    r = _ffi.lib().ecd_layer_stack_layers_per_launch(
        int(nl), int(M), int(D), int(F), int(Hq), int(Hk), int(HD), int(L),
        (2 if stream else 0) | (8 if kv_nt else 0))
    return max(int(r), 0)


def layer_stack_plan(layers, M, D, F, Hq, Hk, HD, dev):
    """The device plan of a layer stack: ``layers`` is a list of dicts with the tensors of
    STACK_FIELDS (n1, wq, sq, kc, vc, o_next None only for the last layer; ``y``, a [M, N] view
    with 16-byte aligned rows, only in the last layer of a 1024-wide stack: it then ends in a
    codebook head with n1, wq, sq the head's norm, packed weights and scales, and no caches).
    The library checks the records (alignment, every layer but the last running the next layer's
    attention, all outputs disjoint) and copies them to the returned uint8 device tensor."""
    nl = len(layers)
    rec = np.zeros((nl, len(STACK_FIELDS)), np.uint64)
    for i, lay in enumerate(layers):
        for j, f in enumerate(STACK_FIELDS):
            t = lay.get(f)
            rec[i, j] = 0 if t is None else t.data_ptr()
    y = layers[-1].get("y")
    yld = 0 if y is None else y.stride(0)
    if y is not None and (y.stride(1) != 1 or yld % 8 or y.shape[0] != M):
        raise ValueError("layer_stack_plan: y must be [M, N], unit column stride, 16-byte rows")
    nb = int(_ffi.lib().ecd_layer_stack_plan_bytes(nl))
    plan = torch.empty(max(nb, 16), device=dev, dtype=torch.uint8)
    _ffi.call("ecd_layer_stack_plan", rec.ctypes.data, nl, M, D, F, Hq, Hk, HD, yld,
              plan.data_ptr(), stream_ptr(dev))
    return plan


def layer_stack(plan, nl, o, xin, xout, rope, pos, q, sync, err, ws, S, Hq, Hk, L, HD, F,
                eps=1e-5, stream=False, no_wait=False, kv_nt=False, y=None):
    """The nl layer tails of ``plan`` (layer_stack_plan) as one launch: layer 0 starts from o
    [M, Hq * HD] and xin [M, D]; each layer's attention output and result feed the next layer.
    Returns ``xout``, the last layer's output buffer of the plan, or ``y``, the logits of a plan
    that ends in a codebook head (the plan's y).  rope, pos, q, sync, err, ws, ``no_wait`` and
    ``kv_nt`` as for layer_tail (sync, err and ws shared with the stack's other layer-tail
    launches)."""
    dev = _dev(o, "layer_stack")
    M, D = xin.shape
    for t, n in ((o, "o"), (xin, "xin")):
        _f16(t, f"layer_stack {n}")
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise ValueError(f"layer_stack: {n} must be contiguous and 16-byte aligned")
    if o.numel() != M * Hq * HD:
        raise ValueError("layer_stack: o must be [M, Hq * HD]")
    if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
        raise ValueError("layer_stack: pos must be contiguous int64 [M]")
    if q.numel() != M * Hq * HD or not q.is_contiguous():
        raise ValueError("layer_stack: q must be contiguous [M, Hq * HD]")
    if rope.shape[0] < L or rope.shape[1] != HD // 2:
        raise ValueError("layer_stack: rope table must be float32 [>= L, HD/2, 2]")
    if sync.dtype != torch.int32 or sync.numel() < 4096 or sync.data_ptr() % 256:
        raise ValueError("layer_stack: sync must be int32 [>= 4096], 256-byte aligned")
    if err.dtype != torch.int32 or err.numel() < 1:
        raise ValueError("layer_stack: err must be int32 [1]")
    if ws.dtype != torch.float32 or ws.data_ptr() % 16 or \
            ws.numel() * 4 < layer_tail_ws_bytes(D, Hq, Hk, HD):
        raise ValueError("layer_stack: ws must be float32, 16-byte aligned, layer_tail_ws_bytes")
    if plan.dtype != torch.uint8 or plan.numel() < int(_ffi.lib().ecd_layer_stack_plan_bytes(nl)):
        raise ValueError("layer_stack: plan must come from layer_stack_plan for nl layers")
    _ffi.call("ecd_layer_stack", plan.data_ptr(), nl, o.data_ptr(), xin.data_ptr(),
              rope.data_ptr(), pos.data_ptr(), q.data_ptr(), sync.data_ptr(), err.data_ptr(),
              ws.data_ptr(), M, D, F, S, Hq, Hk, L, HD, 0 if y is None else y.shape[1],
              0 if y is None else y.stride(0), float(eps),
              _flags(M, stream) | (4 if no_wait else 0) | (8 if kv_nt else 0), stream_ptr(dev))
    return xout if y is None else y


def layer_head(x, nxt, o_next, F, sync, err, ws, eps=1e-5, stream=False, no_wait=False,
               kv_nt=False):
    """A stack's first layer up to its attention as one launch (app/engine.py:189-204 for layer
    0): rms(x, n1) -> q|k|v -> RoPE -> q and the cache slot, and the decode attention into
    o_next [M, Hq * HD].  ``nxt`` as for layer_tail (that layer's n1, wq, ..., S = 1); F: the
    stack's FFN width; sync, err, ws: the stack's layer_tail buffers; ``no_wait`` and
    ``kv_nt`` as for layer_tail."""
    dev = _dev(x, "layer_head")
    M, D = x.shape
    _f16(x, "layer_head x")
    _f16(o_next, "layer_head o_next")
    n = nxt
    pos, kc = n["pos"], n["kc"]
    S, Hq, Hk, L, HD = n["S"], n["Hq"], n["Hk"], n["L"], n["HD"]
    if not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError("layer_head: x must be contiguous and 16-byte aligned")
    if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_contiguous():
        raise ValueError("layer_head: pos must be contiguous int64 [M]")
    if kc.shape != (kc.shape[0], Hk, L, HD) or kc.shape[0] * S < M or n["vc"].shape != kc.shape:
        raise ValueError("layer_head: caches must be [B, Hk, L, HD] with B * S >= M")
    if n["q"].numel() != M * Hq * HD or not n["q"].is_contiguous():
        raise ValueError("layer_head: q must be contiguous [M, Hq * HD]")
    if n["rope"].shape[0] < L or n["rope"].shape[1] != HD // 2:
        raise ValueError("layer_head: rope table must be float32 [>= L, HD/2, 2]")
    if o_next.numel() != M * Hq * HD or not o_next.is_contiguous() or o_next.data_ptr() % 16:
        raise ValueError("layer_head: o_next must be contiguous [M, Hq * HD]")
    if sync.dtype != torch.int32 or sync.numel() < 4096 or sync.data_ptr() % 256:
        raise ValueError("layer_head: sync must be int32 [>= 4096], 256-byte aligned")
    if err.dtype != torch.int32 or err.numel() < 1:
        raise ValueError("layer_head: err must be int32 [1]")
    if ws.dtype != torch.float32 or ws.data_ptr() % 16 or \
            ws.numel() * 4 < layer_tail_ws_bytes(D, Hq, Hk, HD):
        raise ValueError("layer_head: ws must be float32, 16-byte aligned, layer_tail_ws_bytes")
    _ffi.call("ecd_layer_head", x.data_ptr(), n["n1"].data_ptr(), n["wq"].data_ptr(),
              n["sq"].data_ptr(), n["rope"].data_ptr(), pos.data_ptr(), n["q"].data_ptr(),
              kc.data_ptr(), n["vc"].data_ptr(), o_next.data_ptr(), sync.data_ptr(),
              err.data_ptr(), ws.data_ptr(), M, D, F, S, Hq, Hk, L, HD, float(eps),
              _flags(M, stream) | (4 if no_wait else 0) | (8 if kv_nt else 0), stream_ptr(dev))
    return o_next


def embed_gemv_packed(tok, table, tscale, cb, vocab, wp, s, N, even=None, stream=False, out=None,
                      dense=None):
    """int8_mm(Emb(tok[:, 0] + cb * vocab), w, s); with ``even`` [B, K] the input rows are the
    interleave (even[b], emb[b]) and the output has 2B rows.  ``table`` holds int8 rows scaled by
    ``tscale``, or dense fp16 rows when ``tscale`` is None.  ``out``: a contiguous [M, N] fp16
    destination; ``dense``: the numerics (None: int8_mm's rule, dense for more than 16 rows)."""
    dev = _dev(tok, "embed_gemv_packed")
    if tok.dtype != torch.int64:
        raise TypeError("embed_gemv_packed: tok must be int64")
    if (tscale is None) != (table.dtype == torch.float16) or table.dtype not in (torch.int8, torch.float16):
        raise TypeError("embed_gemv_packed: int8 table with scales, or fp16 table without")
    B = tok.shape[0]
    K = table.shape[1]
    M = 2 * B if even is not None else B
    if even is not None:
        _f16(even, "embed_gemv_packed even")
        if even.shape != (B, K) or not even.is_contiguous() or even.data_ptr() % 16:
            raise ValueError("embed_gemv_packed: even must be contiguous [B, K]")
    if out is not None:
        _f16(out, "embed_gemv_packed out")
        if out.shape != (M, N) or not out.is_contiguous():
            raise ValueError(f"embed_gemv_packed: out must be contiguous [{M}, {N}]")
    y = torch.empty(M, N, device=dev, dtype=torch.float16) if out is None else out
    fl = _flags(M, stream) if dense is None else (int(bool(dense)) | (2 if stream else 0))
    _ffi.call("ecd_embed_gemv_i8p", tok.data_ptr(), tok.stride(0), table.data_ptr(), _ptr(tscale),
              table.shape[0], int(cb), int(vocab), _ptr(even), wp.data_ptr(), s.data_ptr(),
              y.data_ptr(), N, M, N, K, fl, stream_ptr(dev))
    return y
