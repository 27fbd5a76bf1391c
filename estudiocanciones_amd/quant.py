"""Per-row int8 quantiser on the GPU (app/convert_final.py:17-21) and synthetic weights.

``q8_rows`` produces the same int8 codes and bf16 scales as the reference converter
(codes from the unrounded fp32 scale, round half to even, clamp to +-127).
``synthetic_weights`` builds a random-init model in the ``mula_int8.safetensors`` layout
(names of app/convert_final.py:32-47 and app/engine.py:110-114, :249-262), quantised on
the device with that kernel -- there is no network to fetch trained weights.
"""
from __future__ import annotations

import torch

from . import _ffi
from .kernels import stream_ptr

AUDIO_VOCAB = 8197
N_CB = 8


def q8_rows(t: torch.Tensor):
    """t [N, K] (any float dtype, ROCm device) -> (q8 int8 [N, K], s8 bfloat16 [N])."""
    if not t.is_cuda:
        raise RuntimeError("q8_rows runs on a ROCm GPU tensor")
    tf = t.float().contiguous()
    N, K = tf.shape
    q = torch.empty(N, K, device=tf.device, dtype=torch.int8)
    s = torch.empty(N, device=tf.device, dtype=torch.bfloat16)
    _ffi.call("ecd_quantize_rows_i8", tf.data_ptr(), q.data_ptr(), s.data_ptr(), None, N, K,
              stream_ptr(tf.device))
    return q, s


def _stack_shapes(prefix, cfg):
    D, H, Hk = cfg["dim"], cfg["heads"], cfg["kv_heads"]
    hd = D // H
    F = cfg.get("ffn", 8192)
    for i in range(cfg["layers"]):
        pre = f"{prefix}.layers.{i}."
        yield pre + "attn.q_proj.weight", (H * hd, D)
        yield pre + "attn.k_proj.weight", (Hk * hd, D)
        yield pre + "attn.v_proj.weight", (Hk * hd, D)
        yield pre + "attn.output_proj.weight", (D, H * hd)
        yield pre + "mlp.w1.weight", (F, D)
        yield pre + "mlp.w3.weight", (F, D)
        yield pre + "mlp.w2.weight", (D, F)


def _stack_norms(prefix, cfg):
    for i in range(cfg["layers"]):
        yield f"{prefix}.layers.{i}.sa_norm.scale", cfg["dim"]
        yield f"{prefix}.layers.{i}.mlp_norm.scale", cfg["dim"]
    yield f"{prefix}.norm.scale", cfg["dim"]


def weight_shapes(backbone: dict, decoder: dict, text_vocab: int = 1024):
    """(quantised tensors {name: (N, K)}, bf16 tensors {name: shape}) of the file layout."""
    Db, Dd = backbone["dim"], decoder["dim"]
    lin = dict(_stack_shapes("backbone", backbone))
    lin.update(_stack_shapes("decoder", decoder))
    lin["projection.weight"] = (Dd, Db)
    lin["codebook0_head.weight"] = (AUDIO_VOCAB, Db)
    for i in range(N_CB - 1):
        lin[f"audio_head.{i}"] = (AUDIO_VOCAB, Dd)
    lin["audio_embeddings.weight"] = (N_CB * AUDIO_VOCAB, Db)
    lin["text_embeddings.weight"] = (text_vocab, Db)
    dense = {n: (d,) for n, d in _stack_norms("backbone", backbone)}
    dense.update({n: (d,) for n, d in _stack_norms("decoder", decoder)})
    dense["unconditional_text_embedding.weight"] = (1, Db)
    dense["muq_linear.bias"] = (Db,)
    return lin, dense


@torch.no_grad()
def synthetic_weights(backbone: dict, decoder: dict, device="cuda", seed: int = 0,
                      std: float = 0.02, emb_std: float = 1.0, text_vocab: int = 1024):
    """Random-init weights in the int8 file layout: linear weights ~ N(0, std), embedding
    tables ~ N(0, emb_std), norm scales 1 + N(0, 0.02), quantised per row on the GPU."""
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    lin, dense = weight_shapes(backbone, decoder, text_vocab)
    out = {}
    for name, (N, K) in lin.items():
        sd = emb_std if "embeddings" in name else std
        w = torch.randn(N, K, generator=g, device=dev) * sd
        out[name + ".q8"], out[name + ".s8"] = q8_rows(w)
        del w
    for name, shp in dense.items():
        if name.endswith(".scale"):
            t = 1.0 + 0.02 * torch.randn(*shp, generator=g, device=dev)
        else:
            t = torch.randn(*shp, generator=g, device=dev) * (emb_std if "embedding" in name else std)
        out[name] = t.to(torch.bfloat16)
    return out
