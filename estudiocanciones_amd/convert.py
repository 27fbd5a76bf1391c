"""Writer of the ``mula_int8.safetensors`` distribution format from the official fp32
HeartMuLa checkpoint (format of app/convert_final.py:17-47, read by app/engine.py:229-265).

Every 2-D tensor becomes per-row int8 codes ``<name>.q8`` plus bf16 scales ``<name>.s8``,
quantised on the GPU by the same kernel the engine uses (``quant.q8_rows``: codes from the
unrounded fp32 scale max|w|/127, round half to even, clamp to +-127).  The stacked
``audio_head`` [7, D, V] is stored as 7 transposed [V, D] heads ``audio_head.{i}``.  The rotary
``pos_embeddings`` (recomputed at load) and ``muq_linear.weight`` (its input is always zero, only
the bias matters) are dropped; ``unconditional_text_embedding.weight`` and every 1-D tensor are
kept in bf16, and with ``--keep-emb-bf16`` the ``text_embeddings`` / ``audio_embeddings`` tables
too (app/convert_final.py:43, :66).  The file metadata carries
``{"lite": "{\\"mode\\": \\"int8\\"}"}``.

    python -m estudiocanciones_amd.convert <HeartMuLa dir | model.safetensors> <out.safetensors>
        [--keep-emb-bf16]
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

from .quant import q8_rows

DROPPED = ("muq_linear.weight",)
KEPT_DENSE = ("unconditional_text_embedding.weight",)


def _dropped(name: str) -> bool:
    return "pos_embeddings" in name or name in DROPPED


def _quantise(t: torch.Tensor, device) -> tuple[torch.Tensor, torch.Tensor]:
    q, s = q8_rows(t.to(device=device, dtype=torch.float32))
    return q.cpu(), s.cpu()


def convert_tensors(items, device="cuda", keep_emb=False) -> dict:
    """(name, tensor) pairs of the official checkpoint -> {name: tensor} of the int8 format;
    ``keep_emb`` keeps the embedding tables in bf16."""
    dev = torch.device(device)
    out = {}
    for name, t in items:
        if _dropped(name):
            continue
        if name == "audio_head":
            for i in range(t.shape[0]):
                out[f"audio_head.{i}.q8"], out[f"audio_head.{i}.s8"] = _quantise(t[i].t(), dev)
        elif t.dim() == 2 and name not in KEPT_DENSE and not (keep_emb and "embeddings" in name):
            out[name + ".q8"], out[name + ".s8"] = _quantise(t, dev)
        else:
            out[name] = t.to(torch.bfloat16).contiguous().cpu()
    return out


def checkpoint_files(src) -> list[Path]:
    """The safetensors shards of a checkpoint directory (index json) or a single file."""
    src = Path(src)
    if src.is_file():
        return [src]
    index = src / "model.safetensors.index.json"
    if index.exists():
        with open(index) as f:
            return [src / n for n in sorted(set(json.load(f)["weight_map"].values()))]
    return [src / "model.safetensors"]


def convert_file(src, dst, device="cuda", keep_emb=False) -> Path:
    """Convert an official checkpoint (directory or file) into ``dst``."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    def items():
        for shard in checkpoint_files(src):
            with safe_open(str(shard), "pt") as f:
                for k in f.keys():
                    yield k, f.get_tensor(k)

    out = convert_tensors(items(), device, keep_emb)
    dst = Path(dst)
    save_file(out, str(dst), metadata={"lite": json.dumps({"mode": "int8"})})
    return dst


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if a != "--keep-emb-bf16"]
    if len(args) != 2:
        raise SystemExit(__doc__)
    path = convert_file(args[0], args[1], keep_emb="--keep-emb-bf16" in sys.argv)
    print(path.name, round(path.stat().st_size / 1e9, 3), "GB")
