"""The fused sampler kernel against the oracle's restatement of _sample/_guided
(app/engine.py:291-305): exact tokens with injected Exponential draws, greedy at top-k 1,
threshold ties kept, and the Philox draws reproducing the top-k softmax distribution."""
import numpy as np
import pytest

from helpers import rng
from oracle.model import cfg_mix, sample

pytestmark = pytest.mark.gpu

V = 8197


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("N,cfg_on,topk,temp", [(4, True, 50, 1.0), (1, True, 50, 0.7),
                                                (3, False, 50, 1.0), (2, True, 1, 1.0),
                                                (4, True, 8197, 1.3)])
def test_sampler_matches_oracle_with_noise(dev, N, cfg_on, topk, temp):
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    g = rng(100 + N + topk)
    B = 2 * N if cfg_on else N
    for trial in range(6):
        logits = (g.standard_normal((B, V), dtype=np.float32) * 3).astype(np.float16)
        noise = g.exponential(1.0, (N, V)).astype(np.float32)
        lg = cfg_mix(logits, N, 1.5) if cfg_on else logits
        want = sample(lg.astype(np.float32), topk, temp, noise)[:, 0]
        # contiguous rows (odd stride: 2-byte loads) and 128-byte aligned rows (16-byte loads)
        padded = torch.zeros(B, 8256, dtype=torch.float16, device=dev)
        padded[:, :V] = T(logits, dev)
        for lg_t in (T(logits, dev), padded[:, :V]):
            out = torch.full((B,), -1, dtype=torch.int64, device=dev)
            sample_topk(lg_t, N, 1.5, temp, topk, out, noise=T(noise, dev))
            got = out.cpu().numpy()
            assert np.array_equal(got[:N], want), (trial, lg_t.stride(0), got[:N], want)
            if cfg_on:
                assert np.array_equal(got[N:], got[:N])


def _shaped_logits(kind, g, B):
    x = g.standard_normal((B, V), dtype=np.float32)
    if kind == "spread":        # 11 values far above the rest: fewer than k near the maximum
        x[:, g.choice(V, 11, replace=False)] = 30000.0
        x[:, 5] = 60000.0
    elif kind == "negative":    # every logit negative
        x = -20.0 + 3.0 * x
    elif kind == "tail":        # maximum and a tie group in the last indices (past 8192)
        x *= 3.0
        x[:, 8195] = 40.0
        x[:, [8192, 8196, 100]] = 20.0
    elif kind in ("edge_in", "edge_out"):   # 50th largest on / just below the lowest key of
        x = 0.01 * x                        # the 16-digit window under 64.0 (digits of 2 bits)
        x[:, :30] = 64.0
        x[:, 30:60] = 5.0 if kind == "edge_in" else 4.996
    return x.astype(np.float16)


@pytest.mark.parametrize("kind", ["spread", "negative", "tail", "edge_in", "edge_out"])
@pytest.mark.parametrize("topk", [1, 50])
def test_sampler_window_and_fallback(dev, kind, topk):
    """Shapes that put the k-th largest value far below the maximum (the full radix select), in
    negative keys, in the tail slots past 8192, or on / just below the window's lowest key."""
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    g = rng(300 + topk)
    N = 2
    for trial in range(3):
        logits = _shaped_logits(kind, g, 2 * N)
        noise = g.exponential(1.0, (N, V)).astype(np.float32)
        want = sample(cfg_mix(logits, N, 1.5).astype(np.float32), topk, 1.0, noise)[:, 0]
        out = torch.full((2 * N,), -1, dtype=torch.int64, device=dev)
        padded = torch.zeros(2 * N, 8256, dtype=torch.float16, device=dev)
        padded[:, :V] = T(logits, dev)
        sample_topk(padded[:, :V], N, 1.5, 1.0, topk, out, noise=T(noise, dev))
        got = out.cpu().numpy()
        assert np.array_equal(got[:N], want), (kind, trial, got, want)


def test_sampler_threshold_ties_kept(dev):
    """Values equal to the k-th largest stay eligible (mask is logits < thr)."""
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    logits = np.full((1, V), -5.0, np.float16)
    logits[0, [10, 20, 30, 40]] = 2.0            # 4-way tie at the top, top-k = 2
    hits = set()
    g = rng(7)
    for t in range(40):
        noise = g.exponential(1.0, (1, V)).astype(np.float32)
        out = torch.zeros(1, dtype=torch.int64, device=dev)
        sample_topk(T(logits, dev), 1, 1.5, 1.0, 2, out, noise=T(noise, dev))
        hits.add(int(out.item()))
    assert hits <= {10, 20, 30, 40} and len(hits) >= 3


def test_sampler_philox_distribution(dev):
    """4096 draws (64 takes x 64 codebook salts) from one logit row: all inside the top-50 set
    and the empirical distribution within total-variation 0.06 of softmax(top-50)."""
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    Nt = 64
    row = (rng(8).standard_normal(V, dtype=np.float32) * 2).astype(np.float16)
    logits = np.tile(row, (Nt, 1))
    lt = T(logits, dev)
    seed = torch.tensor([12345], dtype=torch.int64, device=dev)
    pos = torch.tensor([777], dtype=torch.int64, device=dev)
    counts = np.zeros(V)
    for salt in range(64):
        out = torch.zeros(Nt, dtype=torch.int64, device=dev)
        sample_topk(lt, Nt, 1.0, 1.0, 50, out, seed=seed, pos=pos, salt=salt)
        np.add.at(counts, out.cpu().numpy(), 1)
    x = row.astype(np.float64)
    thr = np.sort(x)[-50]
    top = np.nonzero(x >= thr)[0]                   # values tied with the 50th stay eligible
    assert 50 <= top.size < 80
    assert counts[np.setdiff1d(np.arange(V), top)].sum() == 0
    p = np.zeros(V)
    p[top] = np.exp(x[top] - x[top].max())
    p /= p.sum()
    tv = 0.5 * np.abs(counts / counts.sum() - p).sum()
    assert tv < 0.06, tv


def test_sampler_seed_and_position_change_draws(dev):
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    Nt = 64
    row = np.zeros(V, np.float16)                   # uniform over the top-k set
    lt = T(np.tile(row, (Nt, 1)), dev)

    def draw(seed, p):
        out = torch.zeros(Nt, dtype=torch.int64, device=dev)
        sample_topk(lt, Nt, 1.0, 1.0, V, out, seed=torch.tensor([seed], device=dev),
                    pos=torch.tensor([p], device=dev), salt=0)
        return out.cpu().numpy()

    a = draw(1, 5)
    assert np.array_equal(a, draw(1, 5))           # reproducible
    assert not np.array_equal(a, draw(2, 5))       # seed matters
    assert not np.array_equal(a, draw(1, 6))       # frame position matters


@pytest.mark.parametrize("N,cfg_on,philox", [(4, True, True), (4, True, False), (3, False, True)])
def test_sampler_next_rows(dev, N, cfg_on, philox):
    """ecd_sample_topk_next: the same tokens as ecd_sample_topk, and row b of x = rows[token of
    row b], bit for bit (cond and uncond rows alike), other rows of x untouched."""
    import torch
    from estudiocanciones_amd.kernels import sample_topk
    g = rng(300 + N)
    B = 2 * N if cfg_on else N
    D = 1024
    rows = T((g.standard_normal((V + 3, D), dtype=np.float32)).astype(np.float16), dev)
    seed = torch.tensor([12345], dtype=torch.int64, device=dev)
    pos = torch.tensor([77], dtype=torch.int64, device=dev)
    for trial in range(4):
        logits = T((g.standard_normal((B, V), dtype=np.float32) * 3).astype(np.float16), dev)
        noise = None if philox else T(g.exponential(1.0, (N, V)).astype(np.float32), dev)
        kw = dict(seed=seed, pos=pos, salt=trial) if philox else dict(noise=noise)
        want = torch.full((B,), -1, dtype=torch.int64, device=dev)
        sample_topk(logits, N, 1.5, 1.0, 50, want, **kw)
        got = torch.full((B,), -1, dtype=torch.int64, device=dev)
        x = torch.full((B + 2, D), 7.0, dtype=torch.float16, device=dev)
        # the token-independent copy: ev rows into the even rows of a [2B, D] buffer
        ev = T(g.standard_normal((B, D), dtype=np.float32).astype(np.float16), dev)
        x2 = torch.full((2 * B, D), 5.0, dtype=torch.float16, device=dev)
        sample_topk(logits, N, 1.5, 1.0, 50, got, rows=rows, x=x, ev=ev, xe=x2[0::2], **kw)
        assert torch.equal(got, want), (trial, got, want)
        assert torch.equal(x[:B], rows[got]), trial
        assert bool((x[B:] == 7.0).all())
        assert torch.equal(x2[0::2], ev) and bool((x2[1::2] == 5.0).all())


@pytest.mark.parametrize("N,cfg_on,p,Hq,Hk,HD,D", [
    (4, True, 2, 8, 2, 128, 1024), (4, True, 7, 8, 2, 128, 1024), (3, False, 5, 8, 2, 128, 1024),
    # head_dim 384 (the reference decoder: 8 q / 4 kv heads, 3072 wide), register form
    (4, True, 2, 8, 4, 384, 3072), (4, True, 7, 8, 4, 384, 3072), (3, False, 4, 8, 4, 384, 3072),
    (2, True, 6, 4, 2, 384, 3072)])
def test_sampler_next_layer0_attention(dev, N, cfg_on, p, Hq, Hk, HD, D):
    """ecd_sample_topk_next with the q|k|v rows: per sampled token, k and v land in cache slot p
    bit for bit (other slots untouched), and o is the decode attention over slots 0 .. p
    (oracle.kernels.decode_attn_out, one split) within the fp16 kernel bar; for head_dim 384,
    o is bit-equal to the standalone short-cache attention kernel on the updated caches."""
    import math
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import sample_topk
    from helpers import assert_close16
    from oracle.kernels import decode_attn_out
    g = rng(400 + 10 * N + p + HD)
    B = 2 * N if cfg_on else N
    L = 8
    NQ = (Hq + 2 * Hk) * HD
    rows = T(g.standard_normal((V, D), dtype=np.float32).astype(np.float16), dev)
    qkv = T(g.standard_normal((V, NQ), dtype=np.float32).astype(np.float16), dev)
    kc0 = g.standard_normal((B, Hk, L, HD), dtype=np.float32).astype(np.float16)
    vc0 = g.standard_normal((B, Hk, L, HD), dtype=np.float32).astype(np.float16)
    kc, vc = T(kc0, dev), T(vc0, dev)
    o = torch.full((B, Hq * HD), 3.0, dtype=torch.float16, device=dev)
    x = torch.empty(B, D, dtype=torch.float16, device=dev)
    logits = T((g.standard_normal((B, V), dtype=np.float32) * 3).astype(np.float16), dev)
    noise = T(g.exponential(1.0, (N, V)).astype(np.float32), dev)
    tok = torch.full((B,), -1, dtype=torch.int64, device=dev)
    sample_topk(logits, N, 1.5, 1.0, 50, tok, noise=noise, rows=rows, x=x, qkv=qkv, kc=kc, vc=vc,
                p=p, o=o)
    want_tok = torch.full((B,), -1, dtype=torch.int64, device=dev)
    sample_topk(logits, N, 1.5, 1.0, 50, want_tok, noise=noise)
    assert torch.equal(tok, want_tok)
    assert torch.equal(x, rows[tok])
    t = tok.cpu().numpy()
    tq = qkv.cpu().numpy()[t]                       # [B, NQ]: q heads | k heads | v heads
    kw, vw = kc0.copy(), vc0.copy()
    kw[:, :, p] = tq[:, Hq * HD:(Hq + Hk) * HD].reshape(B, Hk, HD)
    vw[:, :, p] = tq[:, (Hq + Hk) * HD:].reshape(B, Hk, HD)
    assert np.array_equal(kc.cpu().numpy(), kw) and np.array_equal(vc.cpu().numpy(), vw)
    want = decode_attn_out(tq[:, :Hq * HD], kw, vw, np.full(B, p, np.int64), 1, Hq, Hk, HD,
                           nsplit=1)
    assert_close16(o.cpu().numpy(), want, what=f"folded layer-0 attention p={p} HD={HD}")
    if HD == 384:
        qt = T(np.ascontiguousarray(tq[:, :Hq * HD]), dev)
        pos = torch.full((B,), p, dtype=torch.int64, device=dev)
        o2 = torch.full_like(o, 5.0)
        _ffi.call("ecd_decode_attn", qt.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                  o2.data_ptr(), None, None, None, B, 1, Hq, Hk, L, HD, 1, 1.0 / math.sqrt(HD),
                  torch.cuda.current_stream().cuda_stream)
        assert torch.equal(o, o2), "register form differs from the short-cache kernel"
