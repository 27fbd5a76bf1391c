"""Shared test helpers: seeded inputs and small model weights built with the oracle's
quantiser (so the GPU engine and the oracle read identical int8 codes)."""
from __future__ import annotations

import numpy as np

from oracle.numerics import bf16_bits
from oracle.quant import q8_rows

AUDIO_VOCAB = 8197
N_CB = 8

ATOL = 2e-3   # fp16 kernel outputs: max-abs 2e-3 ...
RTOL = 1e-2   # ... or 1e-2 relative


def rng(seed):
    return np.random.default_rng(seed)


def randn16(seed, *shape, std=1.0):
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16)


def tiny_cfgs(ffn=512):
    bb = dict(layers=2, heads=2, kv_heads=1, max_seq=8192, dim=256, ffn=ffn)
    dec = dict(layers=2, heads=2, kv_heads=1, max_seq=2048, dim=256, ffn=ffn)
    return bb, dec


_WEIGHTS_CACHE = {}


def model_weights_np(backbone, decoder, seed=0, std=0.02, emb_std=1.0, text_vocab=64):
    """Random-init weights in the int8 file layout, quantised by the oracle (numpy).
    Memoised per configuration; callers must not modify the returned arrays."""
    key = (tuple(sorted(backbone.items())), tuple(sorted(decoder.items())), seed, std, emb_std,
           text_vocab)
    if key not in _WEIGHTS_CACHE:
        _WEIGHTS_CACHE[key] = _model_weights_np(backbone, decoder, seed, std, emb_std, text_vocab)
    return _WEIGHTS_CACHE[key]


def _model_weights_np(backbone, decoder, seed, std, emb_std, text_vocab):
    from estudiocanciones_amd.quant import weight_shapes  # pure-python shape table
    g = rng(seed)
    lin, dense = weight_shapes(backbone, decoder, text_vocab)
    out = {}
    for name, (N, K) in lin.items():
        sd = emb_std if "embeddings" in name else std
        w = g.standard_normal((N, K), dtype=np.float32) * np.float32(sd)
        out[name + ".q8"], out[name + ".s8"] = q8_rows(w)
    for name, shp in dense.items():
        if name.endswith(".scale"):
            t = 1.0 + 0.02 * g.standard_normal(shp, dtype=np.float32)
        else:
            t = g.standard_normal(shp, dtype=np.float32) * np.float32(emb_std if "embedding" in name else std)
        out[name] = bf16_bits(t)
    return out


def to_torch(weights_np, dev):
    """numpy file-layout dict -> torch tensors on dev (bf16 bit patterns become bfloat16)."""
    import torch
    out = {}
    for k, v in weights_np.items():
        if v.dtype == np.uint16:
            out[k] = torch.from_numpy(v.astype(np.int16)).view(torch.bfloat16).to(dev)
        else:
            out[k] = torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    return out


def assert_close16(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements outside atol={atol} rtol={rtol}; "
            f"worst at {i}: got {got[i]} want {want[i]} (max abs err {err.max():.3e})")


def assert_within_noise(got, want, want_alt, what="", factor=3.0, atol=ATOL, rtol=RTOL):
    """Bar for deep composites (a 28-layer frame, a whole prompt pass), whose outputs move under
    fp32 re-association alone by more than the per-kernel bar: ``want_alt`` is the oracle
    evaluated with float32 instead of float64 sums.  The GPU's largest error against ``want``,
    and its share of elements outside atol + rtol |want|, must stay within ``factor`` times the
    oracle's own (plus one fp16 ulp at the output scale / 0.1% of the elements, at least 4: on
    a 2048-element cache slot one fp16 rounding step across the bar is 0.05%)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    alt = np.asarray(want_alt, np.float64)
    assert got.shape == want.shape == alt.shape, (got.shape, want.shape, alt.shape)
    eg, en = np.abs(got - want), np.abs(alt - want)
    bound = atol + rtol * np.abs(want)
    ulp = float(np.abs(want).max()) * 2.0 ** -10
    fg, fn = float((eg > bound).mean()), float((en > bound).mean())
    assert eg.max() <= factor * en.max() + ulp, \
        f"{what}: max error {eg.max():.3e} vs oracle re-association {en.max():.3e}"
    assert fg <= factor * fn + max(1e-3, 4.0 / eg.size), \
        f"{what}: {fg:.4%} outside the kernel bar vs oracle re-association {fn:.4%}"


def clear_warmup_timeout(st, what=""):
    """After the eager warm-up of a graph capture (a side stream: the kernels' first dispatch
    there): a layer-tail wait that gave up in it is reported and the gate regions cleared, as
    the engine's capture does (its results are discarded, the replays redo its cache writes).
    The replays themselves must then run without one."""
    e = st.tail_error()
    if e:
        print(f"[warm-up] {what}: a layer-tail wait of the capture's warm-up gave up "
              f"(error word {e:#x}); gate regions cleared", flush=True)
        st.tail_reset()
