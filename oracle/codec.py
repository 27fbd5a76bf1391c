"""Oracle of the codec's flow-matching estimator, Euler solver and code embedding (test
infrastructure only).

Restates, in numpy, the fp16 forward of ``LlamaTransformer`` with ``norm_type="ada_norm_single"``
(app/heartcodec/models/transformer.py:275-396) and ``FlowMatching.solve_euler``
(app/heartcodec/models/flow_matching.py:161-210) as the reference runs them (weights and
activations fp16, app/codec_lite.py:13,27).  Every eager fp16 torch op computes in fp32 and
rounds its result to fp16; each such rounding point is an ``f16(...)`` here.  Products and sums
inside one library call (matmul, convolution, reductions, softmax) are evaluated in float64,
which any fp32 accumulation order of the reference lies within the fp16 output tolerance of.

Weights are a dict of numpy arrays under the reference's parameter names relative to the
estimator (``proj_in.ffn_1.weight``, ``transformer_blocks.3.attn.q_proj.weight``, ...).
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import f16, f32

EPS = 1e-6
SQRT1_3 = 3 ** -0.5


def mlp_hidden(dim: int, multiple_of: int = 256) -> int:
    """LlamaMLP hidden width (transformer.py:170-172)."""
    h = int(2 * (4 * dim) / 3)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


# ---------------------------------------------------------------- elementwise pieces
def silu(x) -> np.ndarray:
    """nn.SiLU on fp16: fp16(x / (1 + exp(-x))) evaluated in fp32 or better."""
    a = np.asarray(x, dtype=np.float16).astype(np.float64)
    return f16(a / (1.0 + np.exp(-a)))


def linear(x, w, b=None) -> np.ndarray:
    """F.linear on fp16: fp16(x @ w^T + b) with wide accumulation."""
    y = np.asarray(x, np.float16).astype(np.float64) @ np.asarray(w, np.float16).astype(np.float64).T
    if b is not None:
        y = y + np.asarray(b, np.float16).astype(np.float64)
    return f16(y)


def rms_norm(x, w, eps=EPS) -> np.ndarray:
    """RMSNorm.forward (transformer.py:15-18) on fp16: every op rounds to fp16."""
    x = np.asarray(x, np.float16)
    sq = f16(f32(x) * f32(x))
    var = f16(sq.astype(np.float64).mean(-1, keepdims=True))
    r = f16(1.0 / np.sqrt(f32(f16(f32(var) + np.float32(eps))).astype(np.float64)))
    n = f16(f32(x) * f32(r))
    return f16(f32(np.asarray(w, np.float16)) * f32(n))


def layer_norm(x, eps=EPS) -> np.ndarray:
    """nn.LayerNorm(elementwise_affine=False) on fp16: fp32 statistics, one rounding
    (transformer.py:333-334)."""
    a = np.asarray(x, np.float16).astype(np.float64)
    mu = a.mean(-1, keepdims=True)
    var = ((a - mu) ** 2).mean(-1, keepdims=True)
    return f16((a - mu) / np.sqrt(var + eps))


def modulate(n, shift, scale) -> np.ndarray:
    """n * (1 + scale) + shift on fp16 tensors (transformer.py:239, :245, :370, :393)."""
    one = f16(np.float32(1.0) + f32(scale))
    return f16(f32(f16(f32(n) * f32(one))) + f32(shift))


# ---------------------------------------------------------------- RoPE
def rope_table(T: int, HD: int):
    """RotaryEmbedding.get_sin_cos in fp16 (transformer.py:28-42): (sin, cos) [T, HD/2]."""
    i = np.arange(0, HD, 2, dtype=np.float32)
    ex = f16(i * np.float32(1.0 / HD))
    p = f16(np.power(np.float32(10000.0), f32(ex)))
    inv = f16(np.float32(1.0) / f32(p))
    t = f16(np.arange(T, dtype=np.float32))
    fr = f16(f32(t)[:, None] * f32(inv)[None, :])
    return f16(np.sin(f32(fr))), f16(np.cos(f32(fr)))


def apply_rope_vec(x, sin, cos) -> np.ndarray:
    """apply_rope_vec (transformer.py:108-119): interleaved pairs (x[2i], x[2i+1]) of
    x [B, H, T, HD] rotated by the fp16 table, every product and sum rounded to fp16."""
    x = np.asarray(x, np.float16)
    x1, x2 = f32(x[..., 0::2]), f32(x[..., 1::2])
    s, c = f32(sin)[None, None], f32(cos)[None, None]
    o1 = f16(f32(f16(x1 * c)) - f32(f16(x2 * s)))
    o2 = f16(f32(f16(x1 * s)) + f32(f16(x2 * c)))
    out = np.empty_like(x)
    out[..., 0::2] = o1
    out[..., 1::2] = o2
    return out


# ---------------------------------------------------------------- attention, MLP, blocks
def sdpa(q, k, v) -> np.ndarray:
    """Non-causal scaled_dot_product_attention (transformer.py:140-147): exact softmax over all
    keys, scale 1/sqrt(HD), fp16 output.  q, k, v [B, H, T, HD]."""
    q64, k64, v64 = (np.asarray(a, np.float16).astype(np.float64) for a in (q, k, v))
    s = q64 @ np.swapaxes(k64, -1, -2) / math.sqrt(q.shape[-1])
    p = np.exp(s - s.max(-1, keepdims=True))
    return f16((p @ v64) / p.sum(-1, keepdims=True))


def attention(p: dict, pre: str, x, H: int, HD: int) -> np.ndarray:
    """LlamaAttention.forward without mask (transformer.py:86-149).  x [B, T, D]."""
    B, T, _ = x.shape

    def heads(a):
        return a.reshape(B, T, H, HD).transpose(0, 2, 1, 3)

    q = heads(linear(x, p[pre + "q_proj.weight"]))
    k = heads(linear(x, p[pre + "k_proj.weight"]))
    v = heads(linear(x, p[pre + "v_proj.weight"]))
    sin, cos = rope_table(T, HD)
    q, k = apply_rope_vec(q, sin, cos), apply_rope_vec(k, sin, cos)
    o = sdpa(q, k, v).transpose(0, 2, 1, 3).reshape(B, T, H * HD)
    return linear(o, p[pre + "o_proj.weight"])


def llama_mlp(p: dict, pre: str, x) -> np.ndarray:
    """LlamaMLP.forward (transformer.py:178-181): down(fp16(silu(gate(x)) * up(x)))."""
    g = silu(linear(x, p[pre + "gate.weight"]))
    u = linear(x, p[pre + "up.weight"])
    return linear(f16(f32(g) * f32(u)), p[pre + "down.weight"])


def block(p: dict, pre: str, x, tmod, H: int, HD: int) -> np.ndarray:
    """LlamaTransformerBlock.forward with use_ada_layer_norm_single (transformer.py:225-249).
    tmod [B, 6 * D]."""
    B, _, D = x.shape
    mods = f16(f32(p[pre + "scale_shift_table"])[None] + f32(tmod).reshape(B, 6, D))
    sh_msa, sc_msa, g_msa, sh_mlp, sc_mlp, g_mlp = (mods[:, i:i + 1] for i in range(6))
    n = modulate(rms_norm(x, p[pre + "attn_norm.weight"]), sh_msa, sc_msa)
    h = attention(p, pre + "attn.", n, H, HD)
    x = f16(f32(x) + f32(f16(f32(g_msa) * f32(h))))
    n = modulate(rms_norm(x, p[pre + "mlp_norm.weight"]), sh_mlp, sc_mlp)
    h = llama_mlp(p, pre + "mlp.", n)
    return f16(f32(x) + f32(f16(f32(g_mlp) * f32(h))))


def project_layer(p: dict, pre: str, x) -> np.ndarray:
    """ProjectLayer with kernel_size 3 (transformer.py:258-272): Conv1d(padding 1) over time on
    x [B, T, Cin] (cross-correlation; the library call rounds, then its bias add rounds), times
    3^-0.5 (rounded), then Linear with bias."""
    w = np.asarray(p[pre + "ffn_1.weight"], np.float16).astype(np.float64)   # [Cout, Cin, 3]
    a = np.asarray(x, np.float16).astype(np.float64)
    B, T, _ = a.shape
    pad = np.zeros((B, T + 2, a.shape[2]))
    pad[:, 1:T + 1] = a
    acc = sum(pad[:, j:j + T] @ w[:, :, j].T for j in range(3))
    y = f16(f32(f16(acc)) + f32(p[pre + "ffn_1.bias"]))
    y = f16(f32(y) * np.float32(SQRT1_3))
    return linear(y, p[pre + "ffn_2.weight"], p[pre + "ffn_2.bias"])


# ---------------------------------------------------------------- timestep path
def timestep_sinusoid(t) -> np.ndarray:
    """PixArtAlphaCombinedFlowEmbeddings.timestep_embedding (transformer.py:408-421) in fp32,
    cast to fp16 (:425).  t [n] fp32 -> [n, 512]."""
    i = np.arange(256, dtype=np.float32)
    fr = np.exp((i * np.float32(-math.log(10000))) * np.float32(1 / 256)).astype(np.float32)
    args = (f32(t)[:, None] * fr[None]).astype(np.float32) * np.float32(1000)
    return f16(np.concatenate([np.cos(args.astype(np.float64)),
                               np.sin(args.astype(np.float64))], -1))


def adaln_single(p: dict, pre: str, t):
    """AdaLayerNormSingleFlow.forward (transformer.py:438-444): (linear(silu(emb)), emb) with
    emb = linear_2(silu(linear_1(sinusoid(t)))) (:447-458)."""
    e = timestep_sinusoid(t)
    e = silu(linear(e, p[pre + "emb.timestep_embedder.linear_1.weight"],
                    p[pre + "emb.timestep_embedder.linear_1.bias"]))
    emb = linear(e, p[pre + "emb.timestep_embedder.linear_2.weight"],
                 p[pre + "emb.timestep_embedder.linear_2.bias"])
    return linear(silu(emb), p[pre + "linear.weight"], p[pre + "linear.bias"]), emb


def final_norm(x, table, emb) -> np.ndarray:
    """norm_out / norm_out_2 with the scale_shift_table modulation (transformer.py:366-370)."""
    m = f16(f32(table)[None] + f32(emb)[:, None])
    return modulate(layer_norm(x), m[:, 0:1], m[:, 1:2])


def estimator(p: dict, cfg: dict, hidden, t) -> np.ndarray:
    """LlamaTransformer.forward (transformer.py:345-396).  hidden [B, T, in_channels] fp16,
    t [B] fp32 -> [B, T, out_channels] fp16.  cfg: heads, head_dim, layers, layers_2."""
    H, HD = cfg["heads"], cfg["head_dim"]
    hidden = np.asarray(hidden, np.float16)
    s = project_layer(p, "proj_in.", hidden)
    tmod, emb = adaln_single(p, "adaln_single.", t)
    for i in range(cfg["layers"]):
        s = block(p, f"transformer_blocks.{i}.", s, tmod, H, HD)
    s = final_norm(s, p["scale_shift_table"], emb)
    x = project_layer(p, "connection_proj.", np.concatenate([hidden, s], -1))
    tmod2, emb2 = adaln_single(p, "adaln_single_2.", t)
    for i in range(cfg["layers_2"]):
        x = block(p, f"transformer_blocks_2.{i}.", x, tmod2, H, 2 * HD)
    x = final_norm(x, p["scale_shift_table_2"], emb2)
    return project_layer(p, "proj_out.", x)


# ---------------------------------------------------------------- Euler solver
def solve_euler(est, x, incontext_x, incontext_length: int, t_span, mu, guidance_scale: float):
    """FlowMatching.solve_euler (flow_matching.py:161-210).  ``est(hidden, t)`` is the
    estimator; x, incontext_x [B, T, C] fp16, mu [B, T, Cmu] fp16, t_span fp32.  Scalars t and
    dt are fp32 device tensors in the reference; their products with fp16 tensors round to fp16."""
    x = np.array(x, np.float16)
    ic = np.asarray(incontext_x, np.float16)
    mu = np.asarray(mu, np.float16)
    t_span = f32(t_span)
    L = int(incontext_length)
    t = t_span[0]
    dt = np.float32(t_span[1] - t_span[0])
    noise = x.copy()
    n = len(t_span)
    for step in range(1, n):
        a = np.float32(np.float32(1) - np.float32(np.float32(1 - 1e-6) * t))
        x[:, :L] = f16(f32(f16(a * f32(noise[:, :L]))) + f32(f16(t * f32(ic[:, :L]))))
        if guidance_scale > 1.0:
            inp = np.concatenate([np.concatenate([x, x], 0), np.concatenate([ic, ic], 0),
                                  np.concatenate([np.zeros_like(mu), mu], 0)], 2)
            d = est(inp, np.full(2 * x.shape[0], t, np.float32))
            u, c = np.split(d, 2, 0)
            d = f16(f32(u) + f32(f16(np.float32(guidance_scale) * f32(f16(f32(c) - f32(u))))))
        else:
            d = est(np.concatenate([x, ic, mu], 2), np.full(x.shape[0], t, np.float32))
        x = f16(f32(x) + f32(f16(dt * f32(d))))
        t = np.float32(t + dt)
        if step < n - 1:
            dt = np.float32(t_span[step + 1] - t)
    return x


def t_span(num_steps: int) -> np.ndarray:
    """torch.linspace(0, 1, num_steps + 1) in fp32 (flow_matching.py:140-142): the first half
    from the start, the second half from the end, as torch's linspace evaluates it."""
    n = num_steps + 1
    step = np.float32(1.0) / np.float32(n - 1)
    half = n // 2
    i = np.arange(n, dtype=np.float32)
    lo = (step * i).astype(np.float32)
    hi = (np.float32(1.0) - (step * (np.float32(n - 1) - i)).astype(np.float32)).astype(np.float32)
    return np.where(np.arange(n) < half, lo, hi).astype(np.float32)


# ---------------------------------------------------------------- synthetic weights
def random_weights(cfg: dict, seed: int = 0) -> dict:
    """Random fp16 estimator weights under the reference's names.  cfg: heads, head_dim,
    in_channels, out_channels, layers, layers_2.  Scales keep activations O(1)."""
    g = np.random.default_rng(seed)
    H, HD = cfg["heads"], cfg["head_dim"]
    D, D2, Cin, Cout = H * HD, 2 * H * HD, cfg["in_channels"], cfg["out_channels"]
    p = {}

    def lin(name, n, k, bias=True, gain=1.0):
        p[name + ".weight"] = f16(g.standard_normal((n, k)) * (gain / math.sqrt(k)))
        if bias:
            p[name + ".bias"] = f16(g.standard_normal(n) * 0.02)

    def conv(name, cout, cin):
        p[name + ".ffn_1.weight"] = f16(g.standard_normal((cout, cin, 3)) / math.sqrt(cin))
        p[name + ".ffn_1.bias"] = f16(g.standard_normal(cout) * 0.02)
        lin(name + ".ffn_2", cout, cout)

    def blk(pre, dim):
        p[pre + "attn_norm.weight"] = f16(1 + 0.1 * g.standard_normal(dim))
        p[pre + "mlp_norm.weight"] = f16(1 + 0.1 * g.standard_normal(dim))
        for nm in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin(pre + "attn." + nm, dim, dim, bias=False)
        F = mlp_hidden(dim)
        lin(pre + "mlp.gate", F, dim, bias=False)
        lin(pre + "mlp.up", F, dim, bias=False)
        lin(pre + "mlp.down", dim, F, bias=False)
        p[pre + "scale_shift_table"] = f16(g.standard_normal((6, dim)) / math.sqrt(dim))

    def ada(pre, dim):
        lin(pre + "emb.timestep_embedder.linear_1", dim, 512)
        lin(pre + "emb.timestep_embedder.linear_2", dim, dim)
        lin(pre + "linear", 6 * dim, dim, gain=0.5)

    conv("proj_in", D, Cin)
    for i in range(cfg["layers"]):
        blk(f"transformer_blocks.{i}.", D)
    for i in range(cfg["layers_2"]):
        blk(f"transformer_blocks_2.{i}.", D2)
    conv("connection_proj", D2, Cin + D)
    p["scale_shift_table"] = f16(g.standard_normal((2, D)) / math.sqrt(D))
    p["scale_shift_table_2"] = f16(g.standard_normal((2, D2)) / math.sqrt(D2))
    conv("proj_out", Cout, D2)
    ada("adaln_single.", D)
    ada("adaln_single_2.", D2)
    return p


# ---------------------------------------------------------------- code embedding
def code_embedding(p: dict, codes, num_quantizers: int = 8) -> np.ndarray:
    """FlowMatching.inference_codes conditioning (flow_matching.py:98-108): codebook rows of every
    quantizer (ResidualVQ.get_codes_from_indices; a code of -1 contributes zeros), their fp16 sum,
    project_out, cond_feature_emb, nearest 2x upsampling in time.  codes [B, Q, Tc] ->
    [B, 2 Tc, dim].  Weights under the names relative to ``flow_matching.``."""
    codes = np.asarray(codes, dtype=np.int64)
    B, Q, Tc = codes.shape
    acc = None
    for q in range(num_quantizers):
        book = np.asarray(p[f"vq_embed.layers.{q}._codebook.embed"], np.float16)
        book = book.reshape(-1, book.shape[-1]).astype(np.float64)
        idx = codes[:, q, :]
        e = book[np.clip(idx, 0, None)] * (idx >= 0)[..., None]
        acc = e if acc is None else acc + e
    summed = f16(acc)                                                  # [B, Tc, Dc]
    h = linear(summed, p["vq_embed.project_out.weight"], p["vq_embed.project_out.bias"])
    h = linear(h, p["cond_feature_emb.weight"], p["cond_feature_emb.bias"])
    return np.repeat(h, 2, axis=1)


def inference_codes(p_fm: dict, p_est: dict, cfg: dict, codes, true_latents, latent_length: int,
                    incontext_length: int, guidance_scale: float, num_steps: int, scenario: str,
                    noise) -> np.ndarray:
    """FlowMatching.inference_codes (flow_matching.py:72-159) with the initial sample ``noise``
    given (the reference draws it from torch's global generator)."""
    mu = code_embedding(p_fm, codes)
    B, T, _ = mu.shape
    masks = np.zeros((B, T), np.int64)
    masks[:, :latent_length] = 2
    if scenario == "other_seg":
        masks[:, :incontext_length] = 1
    zero = np.asarray(p_fm["zero_cond_embedding1"], np.float16)
    mu = f16(f32(f16((masks > 0.5)[..., None] * f32(mu))) + f32(f16((masks < 0.5)[..., None] * f32(zero))))
    sel = ((masks > 0.5) & (masks < 1.5))
    ic = f16(np.asarray(true_latents, np.float16).astype(np.float32) * sel[..., None])
    L = int(sel.sum(-1)[0])
    x = solve_euler(lambda h, t: estimator(p_est, cfg, h, t), noise, ic, L, t_span(num_steps), mu,
                    guidance_scale)
    x[:, :L] = ic[:, :L]
    return x


def random_vq_weights(num_quantizers: int, codebook_size: int, codebook_dim: int, dim: int,
                      seed: int = 0) -> dict:
    """Random fp16 code-embedding weights under the reference's names (relative to
    ``flow_matching.``)."""
    g = np.random.default_rng(seed)
    p = {f"vq_embed.layers.{q}._codebook.embed":
         f16(g.standard_normal((1, codebook_size, codebook_dim)) * 0.5) for q in range(num_quantizers)}
    p["vq_embed.project_out.weight"] = f16(g.standard_normal((dim, codebook_dim)) / math.sqrt(codebook_dim))
    p["vq_embed.project_out.bias"] = f16(g.standard_normal(dim) * 0.02)
    p["cond_feature_emb.weight"] = f16(g.standard_normal((dim, dim)) / math.sqrt(dim))
    p["cond_feature_emb.bias"] = f16(g.standard_normal(dim) * 0.02)
    p["zero_cond_embedding1"] = f16(g.standard_normal(dim))
    return p


def detokenize_latents(p_fm: dict, p_est: dict, cfg: dict, codes, duration: float,
                       num_steps: int, guidance_scale: float, noises) -> list:
    """The latent half of HeartCodec.detokenize (modeling_heartcodec.py:57-167) after
    codec_lite.decode's clamp to [0, 8191] (app/codec_lite.py:71; here [0, V - 1]): codes [Q, Tc]
    -> one latent window per hop.  ``noises`` are the windows' initial samples in order."""
    V = np.asarray(p_fm["vq_embed.layers.0._codebook.embed"]).shape[-2]
    codes = np.clip(np.asarray(codes, np.int64), 0, V - 1)[None]
    min_samples = int(duration * 12.5)
    hop = min_samples // 93 * 80
    ovlp_samples = min_samples - hop
    ovlp_frames = ovlp_samples * 2
    if codes.shape[-1] < min_samples:
        while codes.shape[-1] < min_samples:
            codes = np.concatenate([codes, codes], -1)
        codes = codes[:, :, :min_samples]
    if (codes.shape[-1] - ovlp_frames) % hop > 0:
        len_codes = math.ceil((codes.shape[-1] - ovlp_samples) / float(hop)) * hop + ovlp_samples
        while codes.shape[-1] < len_codes:
            codes = np.concatenate([codes, codes], -1)
        codes = codes[:, :, :len_codes]
    latent_length = int(duration * 25)
    C = cfg["out_channels"]
    out = []
    for w, sinx in enumerate(range(0, codes.shape[-1] - hop + 1, hop)):
        win = codes[:, :, sinx:sinx + min_samples]
        true_latent = np.zeros((1, latent_length, C), np.float16)
        L = 0
        if sinx != 0 and ovlp_frames != 0:
            true_latent[:, :ovlp_frames] = out[-1][:, -ovlp_frames:]
            L = ovlp_frames
        out.append(inference_codes(p_fm, p_est, cfg, win, true_latent, latent_length, L,
                                   guidance_scale, num_steps, "other_seg", noises[w]))
    return out


# ---------------------------------------------------------------- waveform decoder
def weight_norm(v, g) -> np.ndarray:
    """torch.nn.utils.parametrizations.weight_norm, dim 0: w = fp16(v * (g / |v|)), norm over
    all but the first axis (fused kernel: fp32 norm, one rounding)."""
    v64 = np.asarray(v, np.float16).astype(np.float64)
    nrm = np.sqrt((v64.reshape(v64.shape[0], -1) ** 2).sum(-1))
    sc = np.asarray(g, np.float16).astype(np.float64).reshape(-1) / nrm
    return f16(v64 * sc.reshape((-1,) + (1,) * (v64.ndim - 1)))


def conv1d(x, w, b, dilation: int = 1, causal: bool = True) -> np.ndarray:
    """Conv1d of sq_codec.py:32-73 on time-major x [B, T, Cin], w [Cout, Cin, k]: causal left
    padding (k - 1) d, else centred padding (k - 1) d / 2; the library rounds its result, then
    the bias add rounds."""
    a = np.asarray(x, np.float16).astype(np.float64)
    w64 = np.asarray(w, np.float16).astype(np.float64)
    B, T, _ = a.shape
    k = w64.shape[2]
    left = (k - 1) * dilation if causal else (k - 1) * dilation // 2
    right = 0 if causal else (k - 1) * dilation - left
    pad = np.zeros((B, T + left + right, a.shape[2]))
    pad[:, left:left + T] = a
    acc = sum(pad[:, j * dilation:j * dilation + T] @ w64[:, :, j].T for j in range(k))
    return f16(f32(f16(acc)) + f32(b))


def conv_transpose_causal(x, w, b, stride: int) -> np.ndarray:
    """ConvTranspose1d(kernel 2s, stride s) with the trailing s outputs dropped (sq_codec.py:
    76-117): out[i*s + j] += x[i] @ w[:, :, j]; x [B, T, Cin], w [Cin, Cout, 2s]."""
    a = np.asarray(x, np.float16).astype(np.float64)
    w64 = np.asarray(w, np.float16).astype(np.float64)
    B, T, _ = a.shape
    k = w64.shape[2]
    out = np.zeros((B, (T - 1) * stride + k, w64.shape[1]))
    for j in range(k):
        out[:, j:j + (T - 1) * stride + 1:stride] += a @ w64[:, :, j]
    out = out[:, :T * stride]
    return f16(f32(f16(out)) + f32(b))


def prelu(x, a: float) -> np.ndarray:
    """nn.PReLU with one slope on fp16."""
    x32 = f32(x)
    return f16(np.where(x32 < 0, np.float32(a) * x32, x32))


def round9(x) -> np.ndarray:
    """round_func9 (sq_codec.py:368-372) on fp16: fp16(9 x) rounded half to even, then the
    division as a multiply by the fp32 reciprocal of 9."""
    r = np.rint(f32(f16(np.float32(9) * f32(x))))
    return f16((r.astype(np.float32) * np.float32(1 / 9)).astype(np.float32))


def _wn(p, pre):
    if pre + "weight" in p:
        return np.asarray(p[pre + "weight"], np.float16)
    return weight_norm(p[pre + "parametrizations.weight.original1"],
                       p[pre + "parametrizations.weight.original0"])


def scalar_decode(p: dict, cfg: dict, latent) -> np.ndarray:
    """ScalarModel.decode (sq_codec.py:522-526) after detokenize's stereo split
    (modeling_heartcodec.py:176-183), time-major: latent [1, T, S * Cl] -> [S, T * up, bands].
    cfg: latent_hidden_dim, upsample_factors."""
    Cl = cfg["latent_hidden_dim"]
    lat = np.asarray(latent, np.float16)[0]
    T = lat.shape[0]
    S = lat.shape[1] // Cl
    x = round9(lat.reshape(T, S, Cl).transpose(1, 0, 2))
    x = conv1d(x, _wn(p, "decoder.0."), p["decoder.0.bias"], causal=False)
    for i, s in enumerate(cfg["upsample_factors"]):
        pre = f"decoder.{1 + i}."
        x = conv_transpose_causal(x, _wn(p, pre + "up_conv.layer."), p[pre + "up_conv.layer.bias"], s)
        for u, d in enumerate((1, 3, 5, 7, 9)):
            q = f"{pre}convs.{u}."
            h = prelu(conv1d(x, _wn(p, q + "conv1."), p[q + "conv1.bias"], d),
                      float(np.asarray(p[q + "activation1.weight"]).reshape(-1)[0]))
            h = prelu(conv1d(h, _wn(p, q + "conv2."), p[q + "conv2.bias"]),
                      float(np.asarray(p[q + "activation2.weight"]).reshape(-1)[0]))
            x = f16(f32(h) + f32(x))
    n = 1 + len(cfg["upsample_factors"])
    x = np.repeat(x, 2, axis=1)
    x = prelu(conv1d(x, p[f"decoder.{n}.conv.weight"], p[f"decoder.{n}.conv.bias"]),
              float(np.asarray(p[f"decoder.{n}.activation.weight"]).reshape(-1)[0]))
    return conv1d(x, _wn(p, f"decoder.{n + 1}."), p[f"decoder.{n + 1}.bias"])


def random_decoder_weights(cfg: dict, seed: int = 0) -> dict:
    """Random fp16 decoder weights under the reference's names (relative to ``scalar_model.``,
    weight-normed layers as parametrization pairs).  cfg: latent_hidden_dim, init_channel,
    upsample_factors."""
    g = np.random.default_rng(seed)
    p = {}
    ups = cfg["upsample_factors"]
    ch = lambda i: cfg["init_channel"] * 2 ** (len(ups) - i)

    def wnl(pre, shape, fan):
        v = g.standard_normal(shape)
        p[pre + "parametrizations.weight.original1"] = f16(v)
        nrm = np.sqrt((v.reshape(shape[0], -1) ** 2).sum(-1))
        p[pre + "parametrizations.weight.original0"] = f16(
            (nrm / math.sqrt(fan) * (1 + 0.1 * g.standard_normal(shape[0]))).reshape((-1, 1, 1)))

    wnl("decoder.0.", (ch(0), cfg["latent_hidden_dim"], 5), cfg["latent_hidden_dim"] * 5)
    p["decoder.0.bias"] = f16(g.standard_normal(ch(0)) * 0.02)
    for i, s in enumerate(ups):
        pre = f"decoder.{1 + i}."
        wnl(pre + "up_conv.layer.", (ch(i), ch(i + 1), 2 * s), ch(i) * 2)
        p[pre + "up_conv.layer.bias"] = f16(g.standard_normal(ch(i + 1)) * 0.02)
        c = ch(i + 1)
        for u in range(5):
            q = f"{pre}convs.{u}."
            wnl(q + "conv1.", (c, c, 7), c * 7 * 4)
            p[q + "conv1.bias"] = f16(g.standard_normal(c) * 0.02)
            wnl(q + "conv2.", (c, c, 1), c * 4)
            p[q + "conv2.bias"] = f16(g.standard_normal(c) * 0.02)
            p[q + "activation1.weight"] = f16([0.25])
            p[q + "activation2.weight"] = f16([0.2])
    n = 1 + len(ups)
    c = cfg["init_channel"]
    p[f"decoder.{n}.conv.weight"] = f16(g.standard_normal((c, c, 7)) / math.sqrt(c * 7))
    p[f"decoder.{n}.conv.bias"] = f16(g.standard_normal(c) * 0.02)
    p[f"decoder.{n}.activation.weight"] = f16([0.25])
    wnl(f"decoder.{n + 1}.", (1, c, 7), c * 7)
    p[f"decoder.{n + 1}.bias"] = f16(g.standard_normal(1) * 0.02)
    return p


def detokenize(p_fm: dict, p_est: dict, cfg: dict, p_dec: dict, dcfg: dict, codes,
               duration: float, num_steps: int, guidance_scale: float, sample_rate: int,
               noises) -> np.ndarray:
    """HeartCodec.detokenize (modeling_heartcodec.py:57-204): latent windows, the waveform of
    each (scalar_decode), crop, linear crossfade over the overlap in float64 stored in fp16
    (through fp32, as torch's CPU copy rounds), cut to the codes' duration."""
    target_len = int(np.asarray(codes).shape[-1] / 12.5 * sample_rate)
    lats = detokenize_latents(p_fm, p_est, cfg, codes, duration, num_steps, guidance_scale, noises)
    min_samples = int(duration * sample_rate)
    hop = min_samples // 93 * 80
    ovlp = min_samples - hop
    out = None
    for lat in lats:
        cur = scalar_decode(p_dec, dcfg, lat)[..., 0][:, :min_samples]
        if out is None:
            out = cur
        else:
            ramp = np.linspace(0, 1, ovlp)
            win = np.concatenate([ramp, 1 - ramp])
            mix = out[:, -ovlp:].astype(np.float64) * win[-ovlp:] + cur[:, :ovlp].astype(np.float64) * win[:ovlp]
            out = out.copy()
            out[:, -ovlp:] = mix.astype(np.float32).astype(np.float16)
            out = np.concatenate([out, cur[:, ovlp:]], -1)
    return out[:, :target_len]
