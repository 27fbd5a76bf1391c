"""Pins for the oracle's frame composition and frame loop (app/engine.py:307-354, :401-446).

* ``OModel.step`` (the fast path, fp16 rounding points) against ``CpuModel.step``, an
  independent float32 restatement of the reference's slow path: the masked backbone call and
  ``_frame_from_h`` with the depth decoder run as ``Stack.__call__`` over ``dec_mask`` on the
  growing sequence.  Planted slips in the fast-path composition -- the codebook-1 head reading
  the backbone-state row of the first decoder pass ([0::2] for [1::2]), codebook i read by
  audio_head[i] instead of audio_head[i - 1], decoder positions one short -- must fail the
  same comparison.
* the backbone input sum against torch's own ``sum(1, dtype=torch.float16)`` on the CPU.
* the EOS scan and trim of the frame loop against its closed form.
"""
import numpy as np
import pytest

from helpers import model_weights_np, tiny_cfgs
from oracle import kernels as K
from oracle.cpu_path import CpuModel
from oracle.model import OModel, frame_loop_trim

V = 8197
N_CB = 8


def _kl(p_logits, q_logits):
    p = np.asarray(p_logits, np.float64)
    q = np.asarray(q_logits, np.float64)
    lp = p - p.max(-1, keepdims=True)
    lp -= np.log(np.exp(lp).sum(-1, keepdims=True))
    lq = q - q.max(-1, keepdims=True)
    lq -= np.log(np.exp(lq).sum(-1, keepdims=True))
    return float((np.exp(lp) * (lp - lq)).sum(-1).max())


def _compare(model_cls, frames=3, seed=11):
    """Teacher-forced frames of ``model_cls`` (an OModel) against the slow-path restatement.
    Returns (worst |logit error| / logit std, worst per-row KL) over all heads and frames."""
    bb, dec = tiny_cfgs()
    w = model_weights_np(bb, dec, seed=seed)
    om = model_cls(w, bb, dec)
    om.alloc(2, 24)
    cm = CpuModel(w, bb, dec)
    cm.alloc(om.B, 24)
    g = np.random.default_rng(seed)
    tok = g.integers(0, V, (om.B, N_CB))
    err = kl = 0.0
    for f in range(frames):
        forced = g.integers(0, V, (om.B, N_CB))
        _, fast = om.step(tok, f, forced=forced)
        slow = cm.step(tok, f, forced)
        for i in range(N_CB):
            a = np.asarray(fast[i], np.float64)
            b = np.asarray(slow[i], np.float64)
            err = max(err, float(np.abs(a - b).max() / b.std()))
            kl = max(kl, _kl(b, a))
        tok = forced
    return err, kl


def test_fast_frame_agrees_with_slow_path():
    err, kl = _compare(OModel)
    assert err < 1e-2, err          # fp16 rounding points vs float32: ~3e-3 of the logit scale
    assert kl < 1e-5, kl


class _SlipPairRow(OModel):
    @staticmethod
    def _pair_last(h):
        return h[0::2]


class _SlipHeadIndex(OModel):
    def _audio_head(self, i):
        return self.audio_head[i % (N_CB - 1)]


class _SlipDecoderPos(OModel):
    @staticmethod
    def _dec_pos(i):
        return i


@pytest.mark.parametrize("slip", [_SlipPairRow, _SlipHeadIndex, _SlipDecoderPos],
                         ids=["pair-row", "head-index", "decoder-pos"])
def test_planted_composition_slips_fail(slip):
    err, kl = _compare(slip)
    assert err > 0.1 and kl > 1e-3, (slip.__name__, err, kl)


def test_embed_sum_matches_torch_fp16_sum():
    """app/engine.py:348: audio_emb(tok + cb_off).sum(1, dtype=fp16) -- the fp16 row products
    summed by torch's reduction (fp32 accumulator, one rounding); a per-step fp16 sum differs."""
    torch = pytest.importorskip("torch")
    g = np.random.default_rng(3)
    D, B = 512, 16
    q8 = g.integers(-127, 128, (N_CB * V, D)).astype(np.int8)
    s = (g.random(N_CB * V) * 0.05 + 1e-3).astype(np.float16)
    tok = g.integers(0, V, (B, N_CB))
    want = K.embed_sum(q8, s, tok, V)
    idx = torch.from_numpy(tok) + torch.arange(N_CB) * V
    q8t, st = torch.from_numpy(q8), torch.from_numpy(s)
    e = torch.nn.functional.embedding(idx, q8t).to(torch.float16) * \
        torch.nn.functional.embedding(idx, st[:, None])
    got = e.sum(1, dtype=torch.float16).numpy()
    assert np.array_equal(got, want)
    rows = tok + np.arange(N_CB)[None] * V
    ef = K.embed_rows(q8, s, rows)
    acc = ef[:, 0]
    for c in range(1, N_CB):
        acc = (acc.astype(np.float32) + ef[:, c].astype(np.float32)).astype(np.float16)
    assert not np.array_equal(acc, got)


def _trim_closed_form(frames, n_frames, check=25):
    hit = (frames >= 8193).any(-1)                                     # [T + 1, N]
    ends = []
    for c in range(frames.shape[1]):
        t = np.flatnonzero(hit[1:, c])
        ends.append(int(t[0]) + 1 if t.size else None)
    if all(e is not None for e in ends):
        marks = sorted({*range(check, n_frames + 1, check), n_frames})
        ran = next(m for m in marks if m >= max(ends))
    else:
        ran = n_frames
    lens = [e if e is not None else n_frames + 1 for e in ends]
    return lens, ran


@pytest.mark.parametrize("n_frames", [7, 25, 60, 130])
def test_frame_loop_trim_closed_form(n_frames):
    g = np.random.default_rng(n_frames)
    for trial in range(60):
        N = int(g.integers(1, 5))
        frames = g.integers(0, 8193, (n_frames + 1, N, N_CB))
        for c in range(N):
            k = int(g.integers(0, 3))
            for _ in range(k):                                         # 0-2 EOS tokens per take
                t = int(g.integers(0, n_frames + 1))
                frames[t, c, int(g.integers(0, N_CB))] = int(g.integers(8193, 8197))
        if trial == 0:
            frames[0, :, 0] = 8193                                     # frame 0 is never scanned
        out, ran = frame_loop_trim(frames, n_frames)
        lens, ran_cf = _trim_closed_form(frames, n_frames)
        assert ran == ran_cf
        for c in range(N):
            assert out[c].shape == (N_CB, lens[c])
            assert np.array_equal(out[c], frames[: lens[c], c].T)


def test_frame_loop_trim_boundaries():
    """EOS on the first frame, on a check frame and just after it, and a take that never ends."""
    n = 60
    frames = np.zeros((n + 1, 4, N_CB), np.int64)
    for c, t in enumerate((1, 25, 26)):
        frames[t, c, 3] = 8193
    out, ran = frame_loop_trim(frames, n)
    assert [o.shape[1] for o in out] == [1, 25, 26, n + 1] and ran == n
    out, ran = frame_loop_trim(frames[:, :3], n)
    assert [o.shape[1] for o in out] == [1, 25, 26] and ran == 50


def test_torch_cpu_path_agrees_with_numpy_slow_path():
    """The torch restatement of the reference's CPU path (the bench's CPU baseline), run in
    float32, agrees with the numpy slow-path restatement under teacher forcing."""
    torch = pytest.importorskip("torch")
    from oracle.cpu_torch import CpuTorchModel
    from helpers import to_torch
    bb, dec = tiny_cfgs()
    w = model_weights_np(bb, dec, seed=11)
    cm = CpuModel(w, bb, dec)
    tm = CpuTorchModel(to_torch(w, "cpu"), bb, dec, dtype=torch.float32)
    tm.alloc(2, 24)
    cm.alloc(tm.B, 24)
    g = np.random.default_rng(5)
    tok = g.integers(0, V, (tm.B, N_CB))
    for f in range(3):
        forced = g.integers(0, V, (tm.B, N_CB))
        want = cm.step(tok, f, forced)
        got = []
        tm.step(torch.from_numpy(tok), f, forced=torch.from_numpy(forced), logits=got)
        for i in range(N_CB):
            np.testing.assert_allclose(got[i].numpy(), want[i], atol=2e-4, rtol=2e-4)
        tok = forced


def test_torch_cpu_path_samples_in_range():
    """Sampling on the torch CPU path (bf16): tokens inside the vocabulary, cond and uncond rows
    of a take equal."""
    torch = pytest.importorskip("torch")
    from oracle.cpu_torch import CpuTorchModel
    from helpers import to_torch
    bb, dec = tiny_cfgs()
    tm = CpuTorchModel(to_torch(model_weights_np(bb, dec, seed=11), "cpu"), bb, dec)
    tm.alloc(2, 24)
    gen = torch.Generator().manual_seed(0)
    t = tm.step(torch.zeros(tm.B, N_CB, dtype=torch.long), 0, gen=gen)
    assert t.shape == (4, N_CB) and int(t.min()) >= 0 and int(t.max()) < V
    assert torch.equal(t[:2], t[2:])
