"""The committed golden vectors (tests/golden/decode_vectors.npz, made by make_golden.py) are
reproduced by the oracle (CPU) and by the gfx950 kernels (GPU)."""
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close16
from oracle import kernels as K
from oracle.model import cfg_mix, sample
from oracle.quant import q8_rows
from oracle.rope import rope_cache

G = np.load(Path(__file__).resolve().parent / "golden" / "decode_vectors.npz")


def test_oracle_reproduces_golden_vectors():
    q, s = q8_rows(G["q8_w"])
    assert np.array_equal(q, G["q8_q"]) and np.array_equal(s, G["q8_s"])
    for M in (8, 20):
        assert np.array_equal(K.gemv_i8(G[f"gemv_x{M}"], G["gemv_q"], G["gemv_s"], G[f"gemv_r{M}"]), G[f"gemv_y{M}"])
    assert np.array_equal(K.rms(G["rms_x"], G["rms_w"]), G["rms_y"])
    assert np.array_equal(rope_cache(128, 40), G["rope_tab"])
    kc, vc = G["rope_kc0"].copy(), G["rope_vc0"].copy()
    assert np.array_equal(K.rope_kv_write(G["rope_qkv"], G["rope_tab"], G["rope_pos"], kc, vc, 2, 4, 2, 128), G["rope_q"])
    assert np.array_equal(kc, G["rope_kc"]) and np.array_equal(vc, G["rope_vc"])
    o = K.decode_attn_out(G["attn_q"], G["attn_k"], G["attn_v"], G["attn_pos"], 1, 6, 2, 128, nsplit=16)
    assert np.array_equal(o, G["attn_o"])
    assert np.array_equal(K.silu_mul(G["silu_x"]), G["silu_y"])
    tok = sample(cfg_mix(G["smp_logits"], 2, 1.5).astype(np.float32), 50, 1.0, G["smp_noise"])
    assert np.array_equal(tok, G["smp_tok"])


@pytest.mark.gpu
def test_gpu_kernels_reproduce_golden_vectors(dev):
    import torch
    from estudiocanciones_amd import kernels as KK
    from estudiocanciones_amd.engine import rope_cache as g_rope
    from estudiocanciones_amd.quant import q8_rows as g_q8

    def T(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    q, s = g_q8(T(G["q8_w"]))
    assert np.array_equal(q.cpu().numpy(), G["q8_q"])
    assert np.array_equal(s.view(torch.int16).cpu().numpy().view(np.uint16), G["q8_s"])
    for M in (8, 20):
        y = KK.int8_mm(T(G[f"gemv_x{M}"]), T(G["gemv_q"]), T(G["gemv_s"]), T(G[f"gemv_r{M}"]))
        assert_close16(y.cpu().numpy(), G[f"gemv_y{M}"], what=f"golden gemv M={M}")
        wp = KK.pack_i8(T(G["gemv_q"]))
        yp = KK.gemv_packed(T(G[f"gemv_x{M}"]), wp, T(G["gemv_s"]), 96, 256, T(G[f"gemv_r{M}"]))
        assert_close16(yp.cpu().numpy(), G[f"gemv_y{M}"], what=f"golden packed gemv M={M}")
    assert_close16(KK.rms(T(G["rms_x"]), T(G["rms_w"])).cpu().numpy(), G["rms_y"], what="golden rms")
    np.testing.assert_allclose(g_rope(128, 40, device=dev).cpu().numpy(), G["rope_tab"], atol=2e-6)
    kc, vc = T(G["rope_kc0"]), T(G["rope_vc0"])
    qo = torch.empty(4, 4 * 128, dtype=torch.float16, device=dev)
    KK._rope_cache[(4, 6)](T(G["rope_qkv"]), T(G["rope_tab"]), T(G["rope_pos"]), qo, kc, vc, 2, 4, 2, 40, HD=128)
    assert_close16(qo.cpu().numpy(), G["rope_q"], what="golden rope q")
    assert_close16(kc.cpu().numpy(), G["rope_kc"], what="golden k cache")
    assert np.array_equal(vc.cpu().numpy(), G["rope_vc"])
    o = torch.empty(2, 6 * 128, dtype=torch.float16, device=dev)
    pm = torch.empty(2 * 6 * 16, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(2 * 6 * 16, 128, device=dev)
    KK._attn[(2, 2, 16)](T(G["attn_q"]), T(G["attn_k"]), T(G["attn_v"]), T(G["attn_pos"]), o, pm, pl, pa,
                         1, 6, 2, 300, 1 / np.sqrt(128), HD=128, NSPLIT=16)
    KK._attn_combine[(12,)](pm, pl, pa, o, HD=128, NSPLIT=16)
    assert_close16(o.cpu().numpy(), G["attn_o"], what="golden attention")
    y = torch.empty(3, 200, dtype=torch.float16, device=dev)
    KK._silu_mul[(3, 1)](T(G["silu_x"]), y, 200, BLOCK=1024)
    assert_close16(y.cpu().numpy(), G["silu_y"], what="golden silu")
    tok = torch.zeros(4, dtype=torch.int64, device=dev)
    KK.sample_topk(T(G["smp_logits"]), 2, 1.5, 1.0, 50, tok, noise=T(G["smp_noise"]))
    assert np.array_equal(tok.cpu().numpy()[:2], G["smp_tok"][:, 0])
