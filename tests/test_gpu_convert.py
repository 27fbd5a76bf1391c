"""The int8 distribution-format writer (app/convert_final.py:17-47, read by
app/engine.py:229-265): every code and scale equals the oracle's quantiser on the same fp32
weights; names, the transposed per-codebook audio heads, the dropped tensors, the bf16 rest and
the metadata follow the format; and the engine loading the written file computes the same
frame as the engine built from the oracle-quantised tensors."""
import json

import numpy as np
import pytest

from helpers import AUDIO_VOCAB, N_CB, assert_close16, rng, tiny_cfgs, to_torch
from oracle.numerics import bf16_bits
from oracle.quant import q8_rows

pytestmark = pytest.mark.gpu

TEXT_VOCAB = 64


def official_checkpoint(bb, dec, seed=21):
    """fp32 tensors under the official names: linear weights [N, K], the audio heads stacked as
    audio_head [7, D, V], and two tensors the format drops."""
    from estudiocanciones_amd.quant import weight_shapes
    g = rng(seed)
    lin, dense = weight_shapes(bb, dec, TEXT_VOCAB)
    ck, heads = {}, []
    for name, (n, k) in lin.items():
        w = g.standard_normal((n, k), dtype=np.float32) * np.float32(1.0 if "embeddings" in name else 0.02)
        if name.startswith("audio_head."):
            heads.append(w)
        else:
            ck[name] = w
    ck["audio_head"] = np.ascontiguousarray(np.stack([h.T for h in heads]))
    for name, shp in dense.items():
        t = g.standard_normal(shp).astype(np.float32)
        ck[name] = (1 + 0.02 * t) if name.endswith(".scale") else t
    ck["backbone.layers.0.attn.pos_embeddings.cache"] = g.standard_normal((16, 8)).astype(np.float32)
    ck["muq_linear.weight"] = g.standard_normal((bb["dim"], 32)).astype(np.float32)
    return ck, heads


def oracle_format(ck, heads):
    """The expected file contents, quantised by the oracle (numpy)."""
    out = {}
    for name, w in ck.items():
        if name in ("audio_head", "muq_linear.weight") or "pos_embeddings" in name:
            continue
        if w.ndim == 2 and name != "unconditional_text_embedding.weight":
            out[name + ".q8"], out[name + ".s8"] = q8_rows(w)
        else:
            out[name] = bf16_bits(w)
    for i, h in enumerate(heads):
        out[f"audio_head.{i}.q8"], out[f"audio_head.{i}.s8"] = q8_rows(h)
    return out


@pytest.fixture(scope="module")
def converted(tmp_path_factory):
    import torch
    from safetensors.torch import save_file
    from estudiocanciones_amd.convert import convert_file
    bb, dec = tiny_cfgs()
    ck, heads = official_checkpoint(bb, dec)
    d = tmp_path_factory.mktemp("ckpt")
    save_file({k: torch.from_numpy(v) for k, v in ck.items()}, str(d / "model.safetensors"))
    out = convert_file(d, d / "mula_int8.safetensors")
    return bb, dec, out, oracle_format(ck, heads)


def test_file_matches_oracle_quantiser(converted):
    from safetensors import safe_open
    _, _, path, want = converted
    import torch
    with safe_open(str(path), "pt") as f:
        keys = set(f.keys())
        assert keys == set(want), sorted(keys ^ set(want))[:10]
        assert json.loads(f.metadata()["lite"]) == {"mode": "int8"}
        for k in sorted(keys):
            got = f.get_tensor(k)
            if k.endswith(".q8"):
                assert got.dtype == torch.int8 and np.array_equal(got.numpy(), want[k]), k
            else:   # bf16 scales and dense tensors: same bit patterns
                assert got.dtype == torch.bfloat16, k
                assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), want[k]), k


def test_engine_loads_written_file(dev, converted):
    """HeartMuLaLite(path) == HeartMuLaLite(oracle-quantised dict): identical logits."""
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    bb, dec, path, want = converted
    a = HeartMuLaLite(str(path), device=dev, backbone=bb, decoder=dec)
    b = HeartMuLaLite(to_torch(want, dev), device=dev, backbone=bb, decoder=dec)
    g = rng(22)
    for m in (a, b):
        m.alloc(1, 16)
    B = a.B
    tok = torch.from_numpy(g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)).to(dev)
    forced = torch.from_numpy(g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)).to(dev)
    pos = torch.zeros(B, 1, dtype=torch.long, device=dev)
    la, lb = [], []
    a._step(tok, pos, None, 1.5, 50, 1.0, forced=forced, logits_out=la)
    b._step(tok, pos, None, 1.5, 50, 1.0, forced=forced, logits_out=lb)
    for i in range(N_CB):
        assert torch.equal(la[i], lb[i]), f"head {i}"


@pytest.fixture(scope="module")
def converted_dense_emb(tmp_path_factory):
    """The same checkpoint written with --keep-emb-bf16 (app/convert_final.py:43, :66)."""
    import torch
    from safetensors.torch import save_file
    from estudiocanciones_amd.convert import convert_file
    bb, dec = tiny_cfgs()
    ck, heads = official_checkpoint(bb, dec)
    d = tmp_path_factory.mktemp("ckpt_emb")
    save_file({k: torch.from_numpy(v) for k, v in ck.items()}, str(d / "model.safetensors"))
    out = convert_file(d, d / "mula_int8.safetensors", keep_emb=True)
    want = oracle_format(ck, heads)
    for name in ("text_embeddings.weight", "audio_embeddings.weight"):
        del want[name + ".q8"], want[name + ".s8"]
        want[name] = bf16_bits(ck[name])
    return bb, dec, out, want


def test_keep_emb_file_matches_oracle(converted_dense_emb):
    """Embedding tables stay bf16 (bit patterns of the fp32 rounded to nearest even)."""
    import torch
    from safetensors import safe_open
    _, _, path, want = converted_dense_emb
    with safe_open(str(path), "pt") as f:
        assert set(f.keys()) == set(want)
        for k in ("text_embeddings.weight", "audio_embeddings.weight"):
            got = f.get_tensor(k)
            assert got.dtype == torch.bfloat16
            assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), want[k]), k


def test_engine_runs_dense_embedding_file(dev, converted_dense_emb):
    """HeartMuLaLite on a --keep-emb-bf16 file: the backbone's codebook sum, the projection
    prologue and the prompt's text rows read the dense tables; teacher-forced frames match the
    oracle's dense-embedding frame (per-kernel bar)."""
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    from oracle.model import OModel
    bb, dec, path, want = converted_dense_emb
    gm = HeartMuLaLite(str(path), device=dev, backbone=bb, decoder=dec)
    assert gm.audio_emb.w is not None and gm.text_emb.w is not None
    om = OModel(want, bb, dec)
    om.alloc(2, 24)
    gm.alloc(2, 24)
    B = gm.B
    g = rng(23)
    tok = g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)
    for f in range(3):
        forced = g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)
        _, olog = om.step(tok, f, forced=forced)
        glog = []
        gm._step(torch.from_numpy(tok).to(dev), torch.full((B, 1), f, dtype=torch.long, device=dev),
                 None, 1.5, 50, 1.0, forced=torch.from_numpy(forced).to(dev), logits_out=glog)
        for i in range(N_CB):
            assert_close16(glog[i].float().cpu().numpy(), olog[i], what=f"dense emb frame {f} head {i}")
        tok = forced
    text = torch.arange(5, device=dev)
    rows = gm.text_emb(text).cpu().numpy()
    from oracle.numerics import bf16_to_f32, f16
    assert np.array_equal(rows, f16(bf16_to_f32(want["text_embeddings.weight"]))[:5])
