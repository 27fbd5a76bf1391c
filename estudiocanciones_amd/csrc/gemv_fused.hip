// Fused int8 GEMV family on lane-ordered packed weights (gfx950).
//
// Packed layout: the [N, K] int8 matrix (rows optionally permuted, see ecd_pack_i8) is cut
// into 16-row x 64-byte chunks; chunk (tile, c) holds rows 16*tile .. +15, bytes
// 64c .. 64c+63, stored as 1 KB in MFMA lane order: bytes [16l, 16l+16) are row l & 15,
// bytes 64c + 16(l >> 4) .. +15.  Chunks of a tile are contiguous in c, so one wave load
// instruction reads 1 KB of contiguous HBM and hands every lane exactly its A fragment of two
// v_mfma_f32_16x16x32_f16.  Rows beyond N are zero padding.
//
// Numerics are those of ecd_gemv_i8 (reference app/kernels.py:20-37, :46-49): fp32
// accumulation of x * q, then fp16(acc * s) (or dequantise-then-GEMM for dense), fp16 residual.
//
// Prologues (how the B fragment, x[m][k], is produced):
//   PRO_PLAIN  x from memory
//   PRO_RMS    x = fp16(fp16(xr * inv[m]) * nw[k]), inv[m] = 1/sqrt(sum(xr[m]^2)/K + eps)
//              computed per block from the full rows (RMSNorm of app/kernels.py:58-67)
//   PRO_EMBED  x = fp16(fp16(q[row]) * s[row]) of an int8 embedding table, row = tok + cb * V,
//              with optional even rows taken from another tensor (app/engine.py:307-308, :336)
// Epilogues:
//   EPI_STORE  y = fp16(acc * s) (+ res)
//   EPI_ROPE   fused q|k|v output: interleaved RoPE of q and k, q -> q_out, k/v -> cache slot
//              (app/kernels.py:78-107 applied to the fp16 GEMV output)
//   EPI_SILU   rows interleaved (w1 row j at 2j, w3 row j at 2j+1): mm[j] = fp16(fp16(silu(a)) * b)
//              (app/kernels.py:171-180 applied to the fp16 GEMV outputs)
#include "common.h"

namespace ecd {

enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_EMBED = 2 };
enum { EPI_STORE = 0, EPI_ROPE = 1, EPI_SILU = 2 };

struct GemvArgs {
  // prologue
  const f16* x;
  long ldx;
  const f16* nw;
  float eps;
  const int64_t* tok;
  long tok_stride;
  const int8_t* etab;
  const f16* escale;
  long erows;
  int cb;
  int vocab;
  const f16* even;
  // weights
  const int8_t* wp;
  const f16* s;
  int M, N, K;
  int dense;
  // EPI_STORE
  const f16* res;
  long ldr;
  f16* y;
  long ldy;
  // EPI_ROPE
  const float* rope;
  const int64_t* pos;
  f16* q;
  f16* kc;
  f16* vc;
  int S, Hq, Hk, L, HD;
  // EPI_SILU
  f16* mm;
};

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *(const f16x8*)p; }

template <int NT, int KW, int PRO, int EPI, int U>
__global__ __launch_bounds__(KW * 64) void gemv_fused_kernel(const GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int tile0 = blockIdx.x * NT;
  const int n0 = tile0 * 16;
  const int m0 = blockIdx.y * 16;
  const int K = a.K, M = a.M, N = a.N;
  const int nch = K >> 6;
  const int ntiles = (N + 15) >> 4;
  const int c0 = (nch * wv) / KW;
  const int c1 = (nch * (wv + 1)) / KW;
  const bool dense = a.dense != 0;

  const int8_t* wb[NT];
  f16 sw[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tile0 + t, ntiles - 1);
    wb[t] = a.wp + (long)tile * nch * 1024 + 16 * lane;
    sw[t] = dense ? a.s[min(n0 + 16 * t + row, N - 1)] : (f16)0.0f;
  }

  // ---- prologue state for batch row m = m0 + row
  const int m = m0 + row;
  const bool mval = m < M;
  __shared__ float s_inv[16];
  const f16* xp = nullptr;
  const f16* nwp = nullptr;
  const int8_t* ep = nullptr;
  f16 esc = (f16)0.0f;
  if (PRO == PRO_PLAIN || PRO == PRO_RMS) {
    xp = a.x + (long)(mval ? m : 0) * a.ldx + 16 * grp;
    if (PRO == PRO_RMS) nwp = a.nw + 16 * grp;
  } else {
    // embedding rows; with `even`, row m even comes from even[m / 2], odd from the table
    const bool from_even = a.even && ((m & 1) == 0);
    const int b = a.even ? (m >> 1) : m;
    if (mval && from_even) {
      xp = a.even + (long)b * K + 16 * grp;
    } else if (mval) {
      const long t = a.tok[(long)b * a.tok_stride];
      const long r = t + (long)a.cb * a.vocab;
      if (t >= 0 && t < a.vocab && r < a.erows) {
        ep = a.etab + r * K + 16 * grp;
        esc = a.escale[r];
      }
    }
  }

  // first weight loads go out before the RMS statistics so their latency overlaps
  u32x4 pre[U][NT];
  const int cpre = min(c0 + U, c1);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (c0 + u < cpre) pre[u][t] = __builtin_nontemporal_load((const u32x4*)(wb[t] + (long)(c0 + u) * 1024));

  float inv = 0.f;
  if (PRO == PRO_RMS) {
    for (int mm = wv; mm < 16; mm += KW) {
      const int mr = m0 + mm;
      float ss = 0.f;
      if (mr < M) {
        const f16* xr = a.x + (long)mr * a.ldx;
        for (int k = lane * 8; k < K; k += 512) {
          const f16x8 v = ld8(xr + k);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) s_inv[mm] = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    __syncthreads();
    inv = s_inv[row];
  }

  auto xfrag = [&](int c, f16x8& fa, f16x8& fb) {
    if (PRO == PRO_EMBED) {
      if (xp) {
        fa = ld8(xp + (long)c * 64);
        fb = ld8(xp + (long)c * 64 + 8);
      } else if (ep) {
        const u32x4 codes = *(const u32x4*)(ep + (long)c * 64);
        i8x16_to_f16(codes, fa, fb);
        fa = fa * esc;
        fb = fb * esc;
      } else {
        fa = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
        fb = fa;
      }
      return;
    }
    if (!mval) {
      fa = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
      fb = fa;
      return;
    }
    fa = ld8(xp + (long)c * 64);
    fb = ld8(xp + (long)c * 64 + 8);
    if (PRO == PRO_RMS) {
      const f16x8 wa = ld8(nwp + (long)c * 64);
      const f16x8 wb2 = ld8(nwp + (long)c * 64 + 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fa[e] = (f16)((float)fa[e] * inv) * wa[e];
        fb[e] = (f16)((float)fb[e] * inv) * wb2[e];
      }
    }
  };

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto step = [&](const u32x4 (&wr)[NT], const f16x8& fa, const f16x8& fb) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f16x8 wa, wbv;
      i8x16_to_f16(wr[t], wa, wbv);
      if (dense) {
        wa = wa * sw[t];
        wbv = wbv * sw[t];
      }
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wbv, fb, acc[t], 0, 0, 0);
    }
  };

  // consume the prefetched chunks
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (c0 + u < cpre) {
      f16x8 fa, fb;
      xfrag(c0 + u, fa, fb);
      step(pre[u], fa, fb);
    }
  }
  int c = cpre;
  for (; c + U <= c1; c += U) {
    u32x4 wr[U][NT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wr[u][t] = __builtin_nontemporal_load((const u32x4*)(wb[t] + (long)(c + u) * 1024));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      f16x8 fa, fb;
      xfrag(c + u, fa, fb);
      step(wr[u], fa, fb);
    }
  }
  for (; c < c1; ++c) {
    u32x4 wr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) wr[t] = __builtin_nontemporal_load((const u32x4*)(wb[t] + (long)c * 1024));
    f16x8 fa, fb;
    xfrag(c, fa, fb);
    step(wr, fa, fb);
  }

  // ---- epilogue on (tile t, lane l): rows n = nb .. nb + 3 of batch row me
  auto epilogue = [&](int t, int l, const f32x4& acc4) {
    const int me = m0 + (l & 15);
    if (me >= M) return;
    const int nb = n0 + 16 * t + 4 * (l >> 4);
    if (nb >= N) return;
    f16 yv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(nb + r, N - 1);
      yv[r] = (f16)(dense ? acc4[r] : acc4[r] * (float)a.s[n]);
    }
    if (EPI == EPI_STORE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nb + r;
        if (n < N) {
          f16 o = yv[r];
          if (a.res) o = o + a.res[(long)me * a.ldr + n];
          a.y[(long)me * a.ldy + n] = o;
        }
      }
    } else if (EPI == EPI_ROPE) {
      // N = (Hq + 2Hk) * HD, HD % 4 == 0: the four columns sit in one head
      const int HD = a.HD;
      const int h = nb / HD, d = nb - h * HD;
      const long p_raw = a.pos[me];
      const int L = a.L;
      const bool pval = p_raw >= 0 && p_raw < L;
      const long p = p_raw < 0 ? 0 : (p_raw >= L ? L - 1 : p_raw);
      f16x4 o;
      if (h < a.Hq + a.Hk) {
        const float* cs = a.rope + p * HD + d;  // (cos, sin) of pairs d/2 and d/2 + 1
        const float c0f = cs[0], s0f = cs[1], c1f = cs[2], s1f = cs[3];
        const float x0 = (float)yv[0], x1 = (float)yv[1], x2 = (float)yv[2], x3 = (float)yv[3];
        o[0] = (f16)(x0 * c0f - x1 * s0f);
        o[1] = (f16)(x1 * c0f + x0 * s0f);
        o[2] = (f16)(x2 * c1f - x3 * s1f);
        o[3] = (f16)(x3 * c1f + x2 * s1f);
      } else {
        o = (f16x4){yv[0], yv[1], yv[2], yv[3]};
      }
      if (h < a.Hq) {
        *(f16x4*)(a.q + ((long)me * a.Hq + h) * HD + d) = o;
      } else if (pval) {
        const int b = me / a.S;
        const int kh = h < a.Hq + a.Hk ? h - a.Hq : h - a.Hq - a.Hk;
        f16* dst = h < a.Hq + a.Hk ? a.kc : a.vc;
        *(f16x4*)(dst + (((long)b * a.Hk + kh) * L + p) * HD + d) = o;
      }
    } else {  // EPI_SILU: (a_j, b_j, a_j+1, b_j+1) with j = nb / 2
      const int F = N >> 1;
      const int j = nb >> 1;
      f16x2 o;
      const float a0 = (float)yv[0], a1 = (float)yv[2];
      o.x = (f16)(a0 / (1.0f + expf(-a0))) * yv[1];
      o.y = (f16)(a1 / (1.0f + expf(-a1))) * yv[3];
      *(f16x2*)(a.mm + (long)me * F + j) = o;
    }
  };

  if constexpr (KW == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) epilogue(t, lane, acc[t]);
  } else {
    __shared__ f32x4 red[KW][NT][64];
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wv][t][lane] = acc[t];
    __syncthreads();
    for (int idx = threadIdx.x; idx < NT * 64; idx += KW * 64) {
      const int t = idx >> 6, l = idx & 63;
      f32x4 s4 = red[0][t][l];
#pragma unroll
      for (int v = 1; v < KW; ++v) s4 += red[v][t][l];
      epilogue(t, l, s4);
    }
  }
}

// Pack w [N, K] into lane-ordered 16 x 64 tiles.  With `interleave` (N even), packed row 2j is
// source row j and packed row 2j + 1 is source row N/2 + j (w1 | w3 -> pairs).
__global__ __launch_bounds__(256) void pack_i8_kernel(const int8_t* __restrict__ w, int N, int K,
                                                      int interleave, int8_t* __restrict__ out) {
  const int nch = K >> 6;
  const long ntiles = (N + 15) >> 4;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= ntiles * nch * 64) return;
  const int l = (int)(idx & 63);
  const long tc = idx >> 6;
  const int c = (int)(tc % nch);
  const long tile = tc / nch;
  const long r = tile * 16 + (l & 15);
  u32x4 v = (u32x4){0u, 0u, 0u, 0u};
  if (r < N) {
    const long src = interleave ? ((r & 1) ? (N >> 1) + (r >> 1) : (r >> 1)) : r;
    v = *(const u32x4*)(w + src * K + 64L * c + 16 * (l >> 4));
  }
  *(u32x4*)(out + (tile * nch + c) * 1024 + 16 * l) = v;
}

struct Cfg {
  int nt, kw;
};

static Cfg pick(int N, int K) {
  const int ntiles = (N + 15) / 16;
  const int nch = K / 64;
  Cfg c{1, 8};
  if (nch >= 128) c.kw = 16;
  else if (nch <= 16) c.kw = 4;
  if (ntiles >= 768 && nch >= 16) c.nt = 2;
  return c;
}

template <int PRO, int EPI>
static int launch(const GemvArgs& a, Cfg c, hipStream_t st) {
  const int ntiles = (a.N + 15) / 16;
#define ECD_FCASE(NT_, KW_)                                                                      \
  if (c.nt == NT_ && c.kw == KW_) {                                                              \
    dim3 grid((ntiles + NT_ - 1) / NT_, (a.M + 15) / 16);                                        \
    hipLaunchKernelGGL((gemv_fused_kernel<NT_, KW_, PRO, EPI, 4>), grid, dim3(KW_ * 64), 0, st, a); \
    return ecd_launch_status();                                                                  \
  }
  ECD_FCASE(1, 4)
  ECD_FCASE(1, 8)
  ECD_FCASE(1, 16)
  ECD_FCASE(2, 4)
  ECD_FCASE(2, 8)
  ECD_FCASE(2, 16)
#undef ECD_FCASE
  return ECD_ENOTSUP;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace ecd

using namespace ecd;

extern "C" {

long ecd_packed_bytes(int N, int K) { return (long)((N + 15) / 16) * 16 * (long)K; }

int ecd_pack_i8(const void* w, int N, int K, int interleave, void* out, void* stream) {
  if (!w || !out || N <= 0 || K <= 0 || (K % 64) || (interleave && (N & 1)) || !aligned16(w) ||
      !aligned16(out))
    return ECD_EINVAL;
  const long total = (long)((N + 15) / 16) * (K / 64) * 64;
  hipLaunchKernelGGL(pack_i8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const int8_t*)w, N, K, interleave, (int8_t*)out);
  return ecd_launch_status();
}

static int check_common(const GemvArgs& a) {
  if (!a.wp || !a.s || a.M <= 0 || a.N <= 0 || a.K <= 0 || (a.K % 64) || !aligned16(a.wp))
    return ECD_EINVAL;
  return ECD_OK;
}

int ecd_gemv_i8p(const void* x, long ldx, const void* wp, const void* s, const void* res, long ldr,
                 void* y, long ldy, int M, int N, int K, int dense, int nt, int kw, void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.wp = (const int8_t*)wp; a.s = (const f16*)s;
  a.M = M; a.N = N; a.K = K; a.dense = dense;
  a.res = (const f16*)res; a.ldr = ldr; a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !x || !y || ldx < K || (ldx % 8) || !aligned16(x) || ldy < N ||
      (res && ldr < N))
    return ECD_EINVAL;
  Cfg c = pick(N, K);
  if (nt > 0) c.nt = nt;
  if (kw > 0) c.kw = kw;
  return launch<PRO_PLAIN, EPI_STORE>(a, c, (hipStream_t)stream);
}

int ecd_rms_gemv_i8p(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* y, long ldy, int M, int N, int K, int dense,
                     void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.N = N; a.K = K; a.dense = dense;
  a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !x || !nw || !y || ldx < K || (ldx % 8) || !aligned16(x) ||
      !aligned16(nw) || ldy < N)
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_STORE>(a, pick(N, K), (hipStream_t)stream);
}

int ecd_rms_qkv_rope(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, const float* rope, const int64_t* pos, void* q, void* kc,
                     void* vc, int M, int S, int Hq, int Hk, int L, int HD, int K, int dense,
                     void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.K = K; a.dense = dense;
  a.N = (Hq + 2 * Hk) * HD;
  a.rope = rope; a.pos = pos; a.q = (f16*)q; a.kc = (f16*)kc; a.vc = (f16*)vc;
  a.S = S; a.Hq = Hq; a.Hk = Hk; a.L = L; a.HD = HD;
  if (check_common(a) || !x || !nw || !rope || !pos || !q || !kc || !vc || S <= 0 || Hq <= 0 ||
      Hk <= 0 || L <= 0 || HD <= 0 || (HD % 4) || (Hq % Hk) || ldx < K || (ldx % 8) ||
      !aligned16(x) || !aligned16(nw))
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_ROPE>(a, pick(a.N, K), (hipStream_t)stream);
}

int ecd_rms_w13_silu(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* mm, int M, int F, int K, int dense, void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.N = 2 * F; a.K = K;
  a.dense = dense; a.mm = (f16*)mm;
  if (check_common(a) || !x || !nw || !mm || F <= 0 || (F % 2) || ldx < K || (ldx % 8) ||
      !aligned16(x) || !aligned16(nw))
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_SILU>(a, pick(a.N, K), (hipStream_t)stream);
}

int ecd_embed_gemv_i8p(const int64_t* tok, long tok_stride, const void* table, const void* tscale,
                       long trows, int cb, int vocab, const void* even, const void* wp,
                       const void* s, void* y, long ldy, int M, int N, int K, int dense,
                       void* stream) {
  GemvArgs a = {};
  a.tok = tok; a.tok_stride = tok_stride; a.etab = (const int8_t*)table;
  a.escale = (const f16*)tscale; a.erows = trows; a.cb = cb; a.vocab = vocab;
  a.even = (const f16*)even; a.wp = (const int8_t*)wp; a.s = (const f16*)s;
  a.M = M; a.N = N; a.K = K; a.dense = dense; a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !tok || !table || !tscale || !y || tok_stride <= 0 || trows <= 0 ||
      cb < 0 || vocab <= 0 || ldy < N || !aligned16(table) || (even && !aligned16(even)) ||
      (even && (M & 1)))
    return ECD_EINVAL;
  return launch<PRO_EMBED, EPI_STORE>(a, pick(N, K), (hipStream_t)stream);
}

}  // extern "C"
