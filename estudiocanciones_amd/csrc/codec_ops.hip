// Row-wise and element-wise kernels of the codec's flow-matching estimator and its Euler
// solver (app/heartcodec/models/transformer.py, app/heartcodec/models/flow_matching.py:161-210)
// on gfx950.  The reference runs these steps as eager fp16 torch ops: each op computes in fp32
// and rounds its result to fp16, so every kernel here rounds at exactly those points (rnd()).
// The dense layers go through the fp16-weight MFMA GEMM and attention through the prompt
// attention kernel; these kernels are the glue between them.
#include "common.h"

// No multiply-add contraction in this file: fp16(fp32(a * b)) is a correctly rounded fp16
// product, which the compiler is free to emit as a half multiply -- and, with contraction on,
// to fuse into a following add as one fma that skips the product's rounding.
#pragma clang fp contract(off)

namespace ecd {

__device__ __forceinline__ float rnd(float v) { return (float)(f16)v; }

// An fp32 result that is rounded to fp32 before any later rounding to fp16 (torch rounds its
// fp32 opmath result to fp32, then casts).  Without the register barrier the backend may fold
// fp16(a * b) into one mixed-precision fma that rounds the exact product straight to fp16.
__device__ __forceinline__ float mul32(float a, float b) {
  float p = a * b;
  asm("" : "+v"(p));
  return p;
}
__device__ __forceinline__ float add32(float a, float b) {
  float p = a + b;
  asm("" : "+v"(p));
  return p;
}

// 256-thread block sum (fp32); `part` holds 4 floats and is reused only after a barrier.
__device__ __forceinline__ float block_sum256(float v, float* part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return part[0] + part[1] + part[2] + part[3];
}

// ---------------------------------------------------------------- RoPE table
// tab[t, i] = (cos f, sin f) in fp16 with f = fp16(fp16(t) * inv_i),
// inv_i = fp16(1 / fp16(10000 ^ fp16(2i * (1 / HD))))  -- RotaryEmbedding.get_sin_cos
// (transformer.py:28-42) evaluated in the activation dtype (fp16), as the reference does.
__global__ __launch_bounds__(256) void codec_rope_table_kernel(f16x2* __restrict__ tab, int T,
                                                               int HD) {
  const int half = HD >> 1;
  const long n = (long)T * half;
  const float rhd = 1.0f / (float)HD;
  for (long e = blockIdx.x * 256L + threadIdx.x; e < n; e += (long)gridDim.x * 256) {
    const int t = (int)(e / half), i = (int)(e - (long)t * half);
    const float ex = rnd(mul32((float)(2 * i), rhd));
    const float p = rnd(powf(10000.f, ex));
    const float inv = rnd(1.0f / p);
    const float f = rnd(rnd((float)t) * inv);
    tab[e] = (f16x2){(f16)cosf(f), (f16)sinf(f)};
  }
}

// ---------------------------------------------------------------- RoPE to heads
// One block per row r = b * T + t of qkv [R, ldq] holding the q | k | v projections
// (H * HD columns each).  Interleaved pairs (x1, x2) = (x[2i], x[2i+1]) of every q and k head
// become (fp16(fp16(x1 c) - fp16(x2 s)), fp16(fp16(x1 s) + fp16(x2 c))) with (c, s) = tab[t, i]
// (apply_rope_vec, transformer.py:108-122).  q stays in rows [R, H * HD]; k and v go to
// [B, H, T, HD], the layout the attention kernel reads.  HD % 8 == 0.
__global__ __launch_bounds__(256) void codec_rope_heads_kernel(
    const f16* __restrict__ qkv, long ldq, const f16x2* __restrict__ tab, f16* __restrict__ q,
    f16* __restrict__ k, f16* __restrict__ v, int T, int H, int HD) {
  const int r = blockIdx.x;
  const int b = r / T, t = r - b * T;
  const int D = H * HD;
  const f16* src = qkv + (long)r * ldq;
  const f16x2* tr = tab + (long)t * (HD >> 1);
  const int nqk = (2 * D) >> 3;
  for (int i = threadIdx.x; i < nqk; i += 256) {
    const int e = i << 3;
    const bool is_k = e >= D;
    const int c = is_k ? e - D : e;
    const int h = c / HD, d = c - h * HD;
    const f16x8 xv = *(const f16x8*)(src + e);
    const f16x8 cs = *(const f16x8*)(tr + (d >> 1));  // 4 (cos, sin) pairs
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16 a, c;
      rope_pair_f16((float)xv[2 * j], (float)xv[2 * j + 1], (float)cs[2 * j], (float)cs[2 * j + 1],
                    a, c);
      o[2 * j] = a;
      o[2 * j + 1] = c;
    }
    if (!is_k)
      *(f16x8*)(q + (long)r * D + c) = o;
    else
      *(f16x8*)(k + (((long)b * H + h) * T + t) * HD + d) = o;
  }
  const int nv = D >> 3;
  for (int i = threadIdx.x; i < nv; i += 256) {
    const int c = i << 3;
    const int h = c / HD, d = c - h * HD;
    *(f16x8*)(v + (((long)b * H + h) * T + t) * HD + d) = *(const f16x8*)(src + 2 * D + c);
  }
}

// ---------------------------------------------------------------- gated residual + norm + adaLN
// One block per row r of x [R, D] (batch b = r / T).  With h != NULL the gated residual of the
// previous branch is applied first and written back: x = fp16(x + fp16(gate * h)),
// gate = fp16(g_tab + g_tm[b])  (LlamaTransformerBlock.forward, transformer.py:241-242,247-248).
// Then the norm:
//   NORM 0 (RMSNorm, :15-18):   n = fp16(w * fp16(x * fp16(rsqrt(fp16(fp16(mean(fp16(x^2))) + eps)))))
//   NORM 1 (LayerNorm without affine, :333-334): n = fp16((x - mean) * rsqrt(var + eps)), fp32 stats
// and the adaLN modulation y = fp16(fp16(n * fp16(1 + scale)) + shift) with
// shift = fp16(sh_tab + sh_tm[b]), scale = fp16(sc_tab + sc_tm[b])  (:234-239, :366-370).
// g_tm of batch b sits at b * g_ld, sh_tm and sc_tm at b * tm_ld (0: one vector shared by every
// batch entry).
// D % 8 == 0, D <= 4096.
template <int NORM>
__global__ __launch_bounds__(256) void codec_norm_mod_kernel(
    f16* __restrict__ x, const f16* __restrict__ h, const f16* __restrict__ g_tab,
    const f16* __restrict__ g_tm, long g_ld, const f16* __restrict__ w, const f16* __restrict__ sh_tab,
    const f16* __restrict__ sh_tm, const f16* __restrict__ sc_tab, const f16* __restrict__ sc_tm,
    long tm_ld, f16* __restrict__ y, int T, int D, float eps) {
  constexpr int NV = 2;
  __shared__ float part0[4], part1[4];
  const int r = blockIdx.x;
  const long bo = (long)(r / T) * tm_ld;
  f16* xr = x + (long)r * D;
  float v[NV][8];
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int c = (threadIdx.x + u * 256) * 8;
    if (c < D) {
      f16x8 xv = *(const f16x8*)(xr + c);
      if (h) {
        const f16x8 hv = *(const f16x8*)(h + (long)r * D + c);
        const f16x8 gt = *(const f16x8*)(g_tab + c);
        const f16x8 gm = *(const f16x8*)(g_tm + (long)(r / T) * g_ld + c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float g = rnd((float)gt[j] + (float)gm[j]);
          xv[j] = (f16)((float)xv[j] + rnd(g * (float)hv[j]));
        }
        *(f16x8*)(xr + c) = xv;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = (float)xv[j];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = 0.f;
    }
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < NV; ++u)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += NORM == 0 ? rnd(v[u][j] * v[u][j]) : v[u][j];
  s = block_sum256(s, part0);
  float mean = 0.f, mul;
  if (NORM == 0) {
    const float ms = rnd(mul32(s, 1.0f / (float)D));
    mul = rnd(rsqrtf(rnd(add32(ms, eps))));
  } else {
    mean = s / (float)D;
    float q = 0.f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = (threadIdx.x + u * 256) * 8;
        const float dv = v[u][j] - mean;
        q += c < D ? dv * dv : 0.f;
      }
    q = block_sum256(q, part1);
    mul = rsqrtf(q / (float)D + eps);
  }
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int c = (threadIdx.x + u * 256) * 8;
    if (c >= D) continue;
    const f16x8 st = *(const f16x8*)(sh_tab + c);
    const f16x8 sm = *(const f16x8*)(sh_tm + bo + c);
    const f16x8 ct = *(const f16x8*)(sc_tab + c);
    const f16x8 cm = *(const f16x8*)(sc_tm + bo + c);
    f16x8 wv;
    if (NORM == 0) wv = *(const f16x8*)(w + c);
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float n;
      if (NORM == 0)
        n = rnd((float)wv[j] * rnd(v[u][j] * mul));
      else
        n = rnd(mul32(v[u][j] - mean, mul));
      const float shift = rnd((float)st[j] + (float)sm[j]);
      const float scale1 = rnd(1.0f + rnd((float)ct[j] + (float)cm[j]));
      o[j] = (f16)(rnd(n * scale1) + shift);
    }
    *(f16x8*)(y + (long)r * D + c) = o;
  }
}

// ---------------------------------------------------------------- k = 3 convolution columns
// Channel segments of the convolution input: segment i contributes w[i] channels read from
// p[i] + ((b % bmod[i]) * (T / rep[i]) + s / rep[i]) * ld[i] for batch entries b >= bzero[i],
// zeros below (rep 2: a half-rate source repeated, nearest 2x upsampling).
struct ColSegs {
  const f16* p[4];
  long ld[4];
  int w[4];
  int bmod[4];
  int bzero[4];
  int rep[4];
  int n;
};

// One block per output row r = b * T + t of cols [R, 3 * C]:
//   cols[r, j * C + c] = in[b, t + j - 1, c]   (zero for t + j - 1 outside [0, T)),
// with in[b, s, :] the concatenation of the segments.  cols @ W'^T with
// W'[o, j * C + c] = conv.weight[o, c, j] is nn.Conv1d(k = 3, padding = 1) of ProjectLayer
// (transformer.py:258-272); the segments express the channel concatenations feeding it
// (solve_euler's [x | incontext | 0 or mu] over [uncond; cond] halves,
// flow_matching.py:183-193, and torch.cat([hidden_states, s]), transformer.py:372).
__global__ __launch_bounds__(256) void codec_cols3_kernel(ColSegs sg, f16* __restrict__ out,
                                                          int T, int C) {
  const int r = blockIdx.x;
  const int b = r / T, t = r - b * T;
  f16* o = out + (long)r * 3 * C;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int s = t + j - 1;
    const bool inside = s >= 0 && s < T;
    int base = j * C;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (g >= sg.n) break;
      const bool live = inside && b >= sg.bzero[g];
      const int rp = sg.rep[g];
      const f16* src =
          sg.p[g] + ((long)(b % sg.bmod[g]) * (T / rp) + (inside ? s : 0) / rp) * sg.ld[g];
      const int nv = sg.w[g] >> 3;
      for (int i = threadIdx.x; i < nv; i += 256) {
        u32x4 val = {0u, 0u, 0u, 0u};
        if (live) val = *(const u32x4*)(src + 8 * i);
        *(u32x4*)(o + base + 8 * i) = val;
      }
      base += sg.w[g];
    }
  }
}

// ---------------------------------------------------------------- code embedding
// out[b * Tc + t, d] = fp16(sum_q codebooks[q, codes[b, q, t], d]) for d < Dc (fp32 sum in
// quantizer order), zero for Dc <= d < Wp: ResidualVQ.get_codes_from_indices then the sum over
// quantizers (flow_matching.py:98-99).  clamp 0: a code of -1 (the library's padding) or any
// code outside [0, V) contributes nothing; clamp 1: codes are first clamped to [0, V - 1], as
// codec_lite.decode does before detokenizing (app/codec_lite.py:71).  codes [B, Q, Tc] int64
// with strides (cb, cq, 1).  One thread per (row, 8 dims).
__global__ __launch_bounds__(256) void codec_vq_embed_kernel(
    const int64_t* __restrict__ codes, long cb, long cq, const f16* __restrict__ books,
    f16* __restrict__ out, int B, int Q, int Tc, int V, int Dc, int Wp, int clamp) {
  const long n = (long)B * Tc * (Wp >> 3);
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int dv = (int)(i % (Wp >> 3)) * 8;
    const long row = i / (Wp >> 3);
    const int b = (int)(row / Tc), t = (int)(row - (long)b * Tc);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (dv < Dc) {
      for (int qq = 0; qq < Q; ++qq) {
        int64_t c = codes[b * cb + qq * cq + t];
        if (clamp) c = c < 0 ? 0 : (c >= V ? V - 1 : c);
        if (c < 0 || c >= V) continue;
        const f16x8 e = *(const f16x8*)(books + ((long)qq * V + c) * Dc + dv);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += (float)e[j];
      }
    }
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (f16)acc[j];
    *(f16x8*)(out + row * Wp + dv) = o;
  }
}

// ---------------------------------------------------------------- waveform decoder glue
// Tap offsets of one convolution (up to 8 taps).
struct Taps {
  int off[8];
  int k;
};

// Tap columns, time-major, for global rows row0 .. row0 + nrows - 1 (row = b * T + t):
// out[row - row0, j * C + c] = src[b, (t + off[j]) / rep, c] when 0 <= t + off[j] < T, else 0.
// src [B, spad + T / rep, C] with row stride ld (spad rows before each sequence, skipped).
// A Conv1d of kernel k and dilation d is the GEMM of these columns with
// W'[o, j * C + c] = weight[o, c, j]:
// causal (sq_codec.py:32-73) off[j] = (j - k + 1) d; centred off[j] = j - (k - 1) / 2; the causal
// ConvTranspose1d (kernel 2s, stride s, sq_codec.py:76-117) uses taps {0, -1}; rep 2 is the
// PostProcessor's nearest 2x repeat (sq_codec.py:140-146).  One thread per 16-byte piece.
__global__ __launch_bounds__(256) void codec_cols_taps_kernel(const f16* __restrict__ src, long ld,
                                                              Taps tp, f16* __restrict__ out,
                                                              int T, int C, int rep, int spad,
                                                              long row0, long nrows) {
  const int vpr = tp.k * C >> 3;  // 16-byte pieces per output row
  const long n = nrows * vpr;
  const int Ts = T / rep;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const long lr = i / vpr;
    const int v = (int)(i - lr * vpr);
    const long row = row0 + lr;
    const int e = v * 8, j = e / C, c = e - j * C;
    const int b = (int)(row / T), t = (int)(row - (long)b * T);
    const int u = t + tp.off[j];
    u32x4 val = {0u, 0u, 0u, 0u};
    if (u >= 0 && u < T)
      val = *(const u32x4*)(src + ((long)b * (Ts + spad) + spad + u / rep) * ld + c);
    *(u32x4*)(out + lr * (long)tp.k * C + e) = val;
  }
}

// Weight normalisation of R rows of n contiguous values (dim 0 of the parametrisation:
// a Conv1d's output channels, a ConvTranspose1d's input channels): w = fp16(v * (g / |v|)) with
// the norm in fp32, as the fused weight-norm kernel computes it (sq_codec.py:152-160,
// torch.nn.utils.parametrizations.weight_norm).
__global__ __launch_bounds__(256) void codec_weight_norm_kernel(const f16* __restrict__ v,
                                                                const f16* __restrict__ g,
                                                                f16* __restrict__ w, int n) {
  __shared__ float part[4];
  const f16* vr = v + (long)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float a = (float)vr[i];
    ss += a * a;
  }
  ss = block_sum256(ss, part);
  const float sc = (float)g[blockIdx.x] / sqrtf(ss);
  for (int i = threadIdx.x; i < n; i += 256) w[(long)blockIdx.x * n + i] = (f16)((float)vr[i] * sc);
}

// The latent of one window [T, S * Cl] (one batch item) split into S channel groups and
// quantised: out[s, t, c] = fp16(fp16(round(fp16(9 x))) * fp32(1 / 9)), x = lat[t, s * Cl + c]
// (modeling_heartcodec.py:176-183 reshape, ScalarModel.decode's round_func9,
// sq_codec.py:368-372, 522-523; the division by 9 is a multiply by the fp32 reciprocal).
__global__ __launch_bounds__(256) void codec_latent_split_kernel(const f16* __restrict__ lat,
                                                                 f16* __restrict__ out, int T,
                                                                 int S, int Cl) {
  const long n = (long)T * S * Cl;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int c = (int)(i % Cl);
    const long tsr = i / Cl;
    const int s = (int)(tsr % S);
    const long t = tsr / S;
    const float x9 = rnd(9.0f * (float)lat[i]);
    const float r = __builtin_rintf(x9);  // round half to even
    out[((long)s * T + t) * Cl + c] = (f16)mul32(r, 1.0f / 9.0f);
  }
}

// ---------------------------------------------------------------- timestep sinusoid
// out[n, i] = cos(a_i), out[n, 256 + i] = sin(a_i) in fp16, a_i = fp32(fp32(t[n] * f_i) * 1000),
// f_i = exp(fp32(i * -ln 10000) * (1 / 256))  -- PixArtAlphaCombinedFlowEmbeddings
// (transformer.py:408-426) with the cast to the hidden dtype.
__global__ __launch_bounds__(256) void codec_timestep_kernel(const float* __restrict__ t,
                                                             f16* __restrict__ out) {
  const int n = blockIdx.x, i = threadIdx.x;
  const float f = expf(((float)i * -9.210340371976184f) * (1.0f / 256.0f));
  const float a = (t[n] * f) * 1000.0f;
  out[(long)n * 512 + i] = (f16)cosf(a);
  out[(long)n * 512 + 256 + i] = (f16)sinf(a);
}

// ---------------------------------------------------------------- SiLU
// y = fp16(x / (1 + exp(-x))) in fp32 (nn.SiLU on fp16 tensors, transformer.py:435,451).
__global__ __launch_bounds__(256) void codec_silu_kernel(const f16* __restrict__ x,
                                                         f16* __restrict__ y, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const float a = (float)x[i];
    y[i] = (f16)(a / (1.0f + expf(-a)));
  }
}

// ---------------------------------------------------------------- Euler step with CFG
// x [B, T, C].  With guidance (cfg 1) dphi is [2B, T, C], unconditional half first
// (flow_matching.py:194), and d = fp16(u + fp16(g * fp16(c - u))) (:195-197); without (cfg 0)
// dphi is [B, T, C] and d = dphi (:199-201).  With dphi: x = fp16(x + fp16(dt * d)) (:203).
// Then rows t < L (the in-context prefix):
//   mode 0: x = fp16(fp16(a * noise) + fp16(tb * ic)), a = fp32(1 - fp32(0.999999 * tb))
//           -- the blend before the next estimator call (:179-181);
//   mode 1: x = ic -- the copy after the last step (:156-158).
// C % 8 == 0.
__global__ __launch_bounds__(256) void codec_euler_kernel(
    f16* __restrict__ x, const f16* __restrict__ noise, const f16* __restrict__ ic,
    const f16* __restrict__ dphi, int cfg, int B, int T, int C, int L, float dt, float g,
    float tb, int mode) {
#pragma clang fp contract(off)
  const long nv = (long)B * T * C >> 3;
  const long half = (long)B * T * C;
  const float a = 1.0f - mul32(0.999999f, tb);
  for (long i = blockIdx.x * 256L + threadIdx.x; i < nv; i += (long)gridDim.x * 256) {
    const long e = i << 3;
    const int t = (int)((e / C) % T);
    f16x8 xv = *(const f16x8*)(x + e);
    if (dphi) {
      const f16x8 u = *(const f16x8*)(dphi + e);
      const f16x8 c = cfg ? *(const f16x8*)(dphi + half + e) : u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float uj = (float)u[j];
        const float d = cfg ? rnd(uj + rnd(mul32(g, rnd((float)c[j] - uj)))) : uj;
        xv[j] = (f16)((float)xv[j] + rnd(mul32(dt, d)));
      }
    }
    if (t < L) {
      const f16x8 icv = *(const f16x8*)(ic + e);
      if (mode == 1) {
        xv = icv;
      } else {
        const f16x8 nz = *(const f16x8*)(noise + e);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xv[j] = (f16)(rnd(mul32(a, (float)nz[j])) + rnd(mul32(tb, (float)icv[j])));
      }
    }
    *(f16x8*)(x + e) = xv;
  }
}

}  // namespace ecd

using namespace ecd;

static inline bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static inline unsigned grid_for(long nthreads) {
  long b = (nthreads + 255) / 256;
  if (b > 8192) b = 8192;
  return (unsigned)(b < 1 ? 1 : b);
}

extern "C" {

int ecd_codec_rope_table(void* tab, int T, int HD, void* stream) {
  if (!tab || T <= 0 || HD <= 0 || (HD & 1)) return ECD_EINVAL;
  hipLaunchKernelGGL(codec_rope_table_kernel, dim3(grid_for((long)T * (HD / 2))), dim3(256), 0,
                     (hipStream_t)stream, (f16x2*)tab, T, HD);
  return ecd_launch_status();
}

int ecd_codec_rope_heads(const void* qkv, long ldq, const void* tab, void* q, void* k, void* v,
                         int B, int T, int H, int HD, void* stream) {
  if (!qkv || !tab || !q || !k || !v || B <= 0 || T <= 0 || H <= 0 || HD <= 0 || (HD & 7) ||
      ldq < 3L * H * HD || (ldq & 7) || !a16(qkv) || !a16(tab) || !a16(q) || !a16(k) || !a16(v))
    return ECD_EINVAL;
  hipLaunchKernelGGL(codec_rope_heads_kernel, dim3(B * T), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)qkv, ldq, (const f16x2*)tab, (f16*)q, (f16*)k, (f16*)v, T, H,
                     HD);
  return ecd_launch_status();
}

int ecd_codec_norm_mod(void* x, const void* h, const void* g_tab, const void* g_tm, long g_ld,
                       const void* w, const void* sh_tab, const void* sh_tm, const void* sc_tab,
                       const void* sc_tm, long tm_ld, void* y, int R, int T, int D, int norm,
                       float eps, void* stream) {
  if (!x || !y || !sh_tab || !sh_tm || !sc_tab || !sc_tm || R <= 0 || T <= 0 || D <= 0 ||
      (D & 7) || D > 4096 || tm_ld < 0 || (tm_ld & 7) || g_ld < 0 || (g_ld & 7) || (norm != 0 && norm != 1) ||
      (norm == 0 && !w) || (h && (!g_tab || !g_tm)))
    return ECD_EINVAL;
  const void* ptrs[] = {x, h, g_tab, g_tm, w, sh_tab, sh_tm, sc_tab, sc_tm, y};
  for (const void* p : ptrs)
    if (p && !a16(p)) return ECD_EINVAL;
  if (norm == 0)
    hipLaunchKernelGGL(codec_norm_mod_kernel<0>, dim3(R), dim3(256), 0, (hipStream_t)stream,
                       (f16*)x, (const f16*)h, (const f16*)g_tab, (const f16*)g_tm, g_ld, (const f16*)w,
                       (const f16*)sh_tab, (const f16*)sh_tm, (const f16*)sc_tab,
                       (const f16*)sc_tm, tm_ld, (f16*)y, T, D, eps);
  else
    hipLaunchKernelGGL(codec_norm_mod_kernel<1>, dim3(R), dim3(256), 0, (hipStream_t)stream,
                       (f16*)x, (const f16*)h, (const f16*)g_tab, (const f16*)g_tm, g_ld, (const f16*)w,
                       (const f16*)sh_tab, (const f16*)sh_tm, (const f16*)sc_tab,
                       (const f16*)sc_tm, tm_ld, (f16*)y, T, D, eps);
  return ecd_launch_status();
}

int ecd_codec_cols3(const void* const* seg_ptr, const long* seg_ld, const int* seg_w,
                    const int* seg_bmod, const int* seg_bzero, const int* seg_rep, int nseg,
                    void* out, int B, int T, void* stream) {
  if (!seg_ptr || !seg_ld || !seg_w || !seg_bmod || !seg_bzero || !out || nseg <= 0 ||
      nseg > 4 || B <= 0 || T <= 0 || !a16(out))
    return ECD_EINVAL;
  ColSegs sg = {};
  int C = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!seg_ptr[i] || !a16(seg_ptr[i]) || seg_w[i] <= 0 || (seg_w[i] & 7) ||
        seg_ld[i] < seg_w[i] || (seg_ld[i] & 7) || seg_bmod[i] <= 0 || seg_bzero[i] < 0 ||
        (seg_rep && (seg_rep[i] <= 0 || T % seg_rep[i])))
      return ECD_EINVAL;
    sg.rep[i] = seg_rep ? seg_rep[i] : 1;
    sg.p[i] = (const f16*)seg_ptr[i];
    sg.ld[i] = seg_ld[i];
    sg.w[i] = seg_w[i];
    sg.bmod[i] = seg_bmod[i];
    sg.bzero[i] = seg_bzero[i];
    C += seg_w[i];
  }
  sg.n = nseg;
  hipLaunchKernelGGL(codec_cols3_kernel, dim3(B * T), dim3(256), 0, (hipStream_t)stream, sg,
                     (f16*)out, T, C);
  return ecd_launch_status();
}

int ecd_codec_vq_embed(const int64_t* codes, long cb, long cq, const void* books, void* out,
                       int B, int Q, int Tc, int V, int Dc, int Wp, int clamp, void* stream) {
  if (!codes || !books || !out || B <= 0 || Q <= 0 || Tc <= 0 || V <= 0 || Dc <= 0 || (Dc & 7) ||
      (clamp != 0 && clamp != 1) ||
      Wp < Dc || (Wp & 7) || cb < 0 || cq < 0 || !a16(books) || !a16(out))
    return ECD_EINVAL;
  hipLaunchKernelGGL(codec_vq_embed_kernel, dim3(grid_for((long)B * Tc * (Wp / 8))), dim3(256), 0,
                     (hipStream_t)stream, codes, cb, cq, (const f16*)books, (f16*)out, B, Q, Tc,
                     V, Dc, Wp, clamp);
  return ecd_launch_status();
}

int ecd_codec_cols_taps(const void* src, long ld, const int* offsets, int k, void* out, int B,
                        int T, int C, int rep, int spad, long row0, long nrows, void* stream) {
  if (!src || !offsets || !out || k <= 0 || k > 8 || B <= 0 || T <= 0 || C <= 0 || (C & 7) ||
      spad < 0 || ld < C || (ld & 7) || (rep != 1 && rep != 2) || T % rep || !a16(src) || !a16(out) ||
      row0 < 0 || nrows <= 0 || row0 + nrows > (long)B * T)
    return ECD_EINVAL;
  Taps tp = {};
  tp.k = k;
  for (int j = 0; j < k; ++j) tp.off[j] = offsets[j];
  hipLaunchKernelGGL(codec_cols_taps_kernel, dim3(grid_for(nrows * (k * C / 8))), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)src, ld, tp, (f16*)out, T, C, rep, spad,
                     row0, nrows);
  return ecd_launch_status();
}

int ecd_codec_weight_norm(const void* v, const void* g, void* w, int rows, int n, void* stream) {
  if (!v || !g || !w || rows <= 0 || n <= 0) return ECD_EINVAL;
  hipLaunchKernelGGL(codec_weight_norm_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)v, (const f16*)g, (f16*)w, n);
  return ecd_launch_status();
}

int ecd_codec_latent_split(const void* lat, void* out, int T, int S, int Cl, void* stream) {
  if (!lat || !out || T <= 0 || S <= 0 || Cl <= 0) return ECD_EINVAL;
  hipLaunchKernelGGL(codec_latent_split_kernel, dim3(grid_for((long)T * S * Cl)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)lat, (f16*)out, T, S, Cl);
  return ecd_launch_status();
}

int ecd_codec_timestep(const float* t, void* out, int n, void* stream) {
  if (!t || !out || n <= 0) return ECD_EINVAL;
  hipLaunchKernelGGL(codec_timestep_kernel, dim3(n), dim3(256), 0, (hipStream_t)stream, t,
                     (f16*)out);
  return ecd_launch_status();
}

int ecd_codec_silu(const void* x, void* y, long n, void* stream) {
  if (!x || !y || n <= 0) return ECD_EINVAL;
  hipLaunchKernelGGL(codec_silu_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)x, (f16*)y, n);
  return ecd_launch_status();
}

int ecd_codec_euler(void* x, const void* noise, const void* ic, const void* dphi, int cfg, int B,
                    int T, int C, int L, float dt, float g, float tb, int mode, void* stream) {
  if (!x || (cfg != 0 && cfg != 1) || B <= 0 || T <= 0 || C <= 0 || (C & 7) || L < 0 || L > T || (mode != 0 && mode != 1) ||
      (L > 0 && (!ic || (mode == 0 && !noise))) || !a16(x) || (ic && !a16(ic)) ||
      (noise && !a16(noise)) || (dphi && !a16(dphi)))
    return ECD_EINVAL;
  hipLaunchKernelGGL(codec_euler_kernel, dim3(grid_for((long)B * T * C / 8)), dim3(256), 0,
                     (hipStream_t)stream, (f16*)x, (const f16*)noise, (const f16*)ic,
                     (const f16*)dphi, cfg, B, T, C, L, dt, g, tb, mode);
  return ecd_launch_status();
}

}  // extern "C"
