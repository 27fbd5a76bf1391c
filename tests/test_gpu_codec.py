"""Kernels of the codec's flow-matching estimator (app/heartcodec/models/transformer.py) against
fp32 numpy products with the same fp16 rounding points as torch's fp16 layers."""
import numpy as np
import pytest

from helpers import assert_close16, randn16, rng
from oracle.numerics import f16

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N_(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("M,N,K,bias,alpha,res", [
    (17, 100, 64, True, 1.0, False),          # ragged M and N, one K chunk
    (1488, 1536, 3072, True, 3 ** -0.5, False),  # ProjectLayer conv (k = 3) as a GEMM, scaled
    (200, 1536, 7680, False, 1.0, True),      # connection_proj width (K = 3 x 2560), residual
    (96, 3072, 1536, True, 1.0, True),
])
def test_gemm_f16_linear(dev, M, N, K, bias, alpha, res):
    """F.linear(x, w, b) numerics: fp32 accumulation and bias, one fp16 rounding; then the
    optional fp16 scale and fp16 residual add."""
    from estudiocanciones_amd.kernels import gemm_f16_packed, pack_f16
    g = rng(400 + K)
    x = randn16(401 + M, M, K)
    w = (g.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
    b = (g.standard_normal(N, dtype=np.float32) * 0.1) if bias else None
    r = randn16(402 + M, M, N) if res else None
    want = x.astype(np.float32) @ w.astype(np.float32).T
    if bias:
        want = want + b
    want = f16(want)
    if alpha != 1.0:
        want = f16(want.astype(np.float32) * np.float32(alpha))
    if res:
        want = f16(want.astype(np.float32) + r.astype(np.float32))
    got = gemm_f16_packed(T(x, dev), pack_f16(T(w, dev)), N, K, T(b, dev) if bias else None,
                          alpha, T(r, dev) if res else None)
    assert_close16(N_(got), want, what=f"gemm f16 M={M} N={N} K={K}")


@pytest.mark.parametrize("M,F,K", [(40, 256, 128), (1488, 4096, 1536)])
def test_gemm_f16_silu(dev, M, F, K):
    """LlamaMLP's F.silu(gate(x)) * up(x) in fp16 (transformer.py:181-184)."""
    from estudiocanciones_amd.kernels import gemm_f16_silu_packed, pack_f16
    import torch
    g = rng(410 + F)
    x = randn16(411 + M, M, K)
    gate = (g.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    up = (g.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    a = f16(x.astype(np.float32) @ gate.astype(np.float32).T).astype(np.float32)
    u = f16(x.astype(np.float32) @ up.astype(np.float32).T).astype(np.float32)
    want = f16(f16(a / (1.0 + np.exp(-a))).astype(np.float32) * u)
    wp = pack_f16(torch.cat([T(gate, dev), T(up, dev)], 0).contiguous(), interleave=True)
    got = gemm_f16_silu_packed(T(x, dev), wp, F, K)
    assert_close16(N_(got), want, what=f"gemm f16 silu M={M} F={F}")
