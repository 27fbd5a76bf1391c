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
//   PRO_EMBED  x = fp16(fp16(q[row]) * s[row]) of an int8 embedding table (or the row of a dense
//              fp16 table), row = tok + cb * V, with optional even rows taken from another
//              tensor (app/engine.py:307-308, :336)
// Epilogues:
//   EPI_STORE  y = fp16(acc * s) (+ res)
//   EPI_ROPE   fused q|k|v output: interleaved RoPE of q and k, q -> q_out, k/v -> cache slot
//              (app/kernels.py:78-107 applied to the fp16 GEMV output)
//   EPI_SILU   rows interleaved (w1 row j at 2j, w3 row j at 2j+1): mm[j] = fp16(fp16(silu(a)) * b)
//              (app/kernels.py:171-180 applied to the fp16 GEMV outputs)
//   EPI_PARTIAL split K: block z writes its fp32 sums to ws[z][M][N]; splitk_reduce_kernel adds
//              the splits in order and applies the scale and residual of EPI_STORE
#include "common.h"

namespace ecd {

enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_EMBED = 2 };
enum { EPI_STORE = 0, EPI_ROPE = 1, EPI_SILU = 2, EPI_PARTIAL = 3 };

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
  const f16* etab16;  // dense fp16 embedding table (etab/escale unused when set)
  long erows;
  int cb;
  int vocab;
  const f16* even;
  // weights
  const int8_t* wp;
  const f16* s;
  int M, N, K;
  int dense;
  int stream_hint;  // 1: weights are streamed once (nontemporal loads), 0: keep them cacheable
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
  int qrows;  // 1: q receives every head of row m as row m of [M, N] (q | k | v), no cache write
  // EPI_SILU
  f16* mm;
  // EPI_PARTIAL: ks K-splits (blockIdx.z), fp32 partial sums [ks][M][N]
  float* ws;
  int ks;
};

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *(const f16x8*)p; }

// Epilogue operands of tile t, lane l (rows n = nb .. nb + 3 of batch row me, the C layout of
// v_mfma_f32_16x16x32_f16: lane l holds rows 4 (l >> 4) + r of column l & 15).  They are
// fetched at kernel start, so the epilogue after the K reduction makes no dependent global
// load: scales, residual, and for the RoPE epilogue the position and its cos/sin pairs.
struct EpiPre {
  f16 s[4];
  f16 r[4];
  float cs[4];
  long p;
};

template <int EPI>
__device__ __forceinline__ EpiPre epi_prefetch(const GemvArgs& a, int n0, int m0, int t, int l) {
  EpiPre e;
  const int me = m0 + (l & 15);
  const int nb = n0 + 16 * t + 4 * (l >> 4);
  const bool ok = me < a.M && nb < a.N;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    e.s[r] = a.s[min(nb + r, a.N - 1)];
    e.r[r] = (f16)0.0f;
    e.cs[r] = 0.f;
  }
  e.p = 0;
  if (EPI == EPI_STORE && a.res && ok) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (nb + r < a.N) e.r[r] = a.res[(long)me * a.ldr + nb + r];
  }
  if (EPI == EPI_ROPE && ok) {
    const int HD = a.HD;
    const int h = nb / HD, d = nb - h * HD;
    const long p_raw = a.pos[me];
    e.p = p_raw;
    if (h < a.Hq + a.Hk) {
      const long pc = p_raw < 0 ? 0 : (p_raw >= a.L ? a.L - 1 : p_raw);
      const float* cs = a.rope + pc * HD + d;  // (cos, sin) of pairs d/2 and d/2 + 1
#pragma unroll
      for (int r = 0; r < 4; ++r) e.cs[r] = cs[r];
    }
  }
  return e;
}

template <int EPI>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, int n0, int m0, int t, int l,
                                              const f32x4& acc4, const EpiPre& e) {
  const int M = a.M, N = a.N;
  const bool dense = a.dense != 0;
  const int me = m0 + (l & 15);
  if (me >= M) return;
  const int nb = n0 + 16 * t + 4 * (l >> 4);
  if (nb >= N) return;
  if constexpr (EPI == EPI_PARTIAL) {
    float* dst = a.ws + ((long)blockIdx.z * M + me) * N + nb;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (nb + r < N) dst[r] = acc4[r];
    return;
  }
  f16 yv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) yv[r] = (f16)(dense ? acc4[r] : acc4[r] * (float)e.s[r]);
  if (EPI == EPI_STORE) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nb + r;
      if (n < N) {
        f16 o = yv[r];
        if (a.res) o = o + e.r[r];
        a.y[(long)me * a.ldy + n] = o;
      }
    }
  } else if (EPI == EPI_ROPE) {
    // N = (Hq + 2Hk) * HD, HD % 4 == 0: the four columns sit in one head
    const int HD = a.HD;
    const int h = nb / HD, d = nb - h * HD;
    const int L = a.L;
    const long p_raw = e.p;
    const bool pval = p_raw >= 0 && p_raw < L;
    const long p = p_raw < 0 ? 0 : (p_raw >= L ? L - 1 : p_raw);
    f16x4 o;
    if (h < a.Hq + a.Hk) {
      const float x0 = (float)yv[0], x1 = (float)yv[1], x2 = (float)yv[2], x3 = (float)yv[3];
      o[0] = (f16)(x0 * e.cs[0] - x1 * e.cs[1]);
      o[1] = (f16)(x1 * e.cs[0] + x0 * e.cs[1]);
      o[2] = (f16)(x2 * e.cs[2] - x3 * e.cs[3]);
      o[3] = (f16)(x3 * e.cs[2] + x2 * e.cs[3]);
    } else {
      o = (f16x4){yv[0], yv[1], yv[2], yv[3]};
    }
    if (a.qrows) {
      *(f16x4*)(a.q + (long)me * N + nb) = o;
    } else if (h < a.Hq) {
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
}

constexpr int NW_MAX = 4096;  // RMS prologue: normalisation weights staged in LDS (K <= NW_MAX)

template <bool NTL>
__device__ __forceinline__ u32x4 ldw(const int8_t* p) {
  if (NTL) return __builtin_nontemporal_load((const u32x4*)p);
  return *(const u32x4*)p;
}

// One wave owns chunks [c0, c1) of every tile of its block and processes them in groups of CW:
// all weight loads of a group are issued back to back (one memory latency per group), then the
// x fragments, then the MFMAs.  Blocks are KW waves splitting K, NT tiles of 16 rows each.
template <int NT, int KW, int PRO, int EPI, int CW, bool NTL>
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
  const f16* xp = nullptr;
  const int8_t* ep = nullptr;
  f16 esc = (f16)0.0f;
  if (PRO == PRO_PLAIN || PRO == PRO_RMS) {
    if (mval) xp = a.x + (long)m * a.ldx + 16 * grp;
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
        if (a.etab16) {
          xp = a.etab16 + r * K + 16 * grp;  // a dense row reads like x
        } else {
          ep = a.etab + r * K + 16 * grp;
          esc = a.escale[r];
        }
      }
    }
  }

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // epilogue operands of this thread's (tile, lane) slot, fetched up front
  const bool epi_thread = (int)threadIdx.x < NT * 64;
  EpiPre pre_e;
  if (KW > 1 && epi_thread) pre_e = epi_prefetch<EPI>(a, n0, m0, threadIdx.x >> 6, threadIdx.x & 63);

  u32x4 wr[CW][NT];
  int cb = c0;
  int nc = min(CW, c1 - cb);
#pragma unroll
  for (int u = 0; u < CW; ++u)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (u < nc) wr[u][t] = ldw<NTL>(wb[t] + (long)(cb + u) * 1024);

  // RMS statistics while the first weight group is in flight
  __shared__ float s_inv[16];
  __shared__ f16 s_nw[PRO == PRO_RMS ? NW_MAX : 8];
  float inv = 0.f;
  if (PRO == PRO_RMS) {
    for (int k = threadIdx.x * 8; k < K; k += KW * 64 * 8) *(f16x8*)(s_nw + k) = ld8(a.nw + k);
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

  while (nc > 0) {
    // raw x fragments of the group
    u32x4 xa[CW], xb[CW];
#pragma unroll
    for (int u = 0; u < CW; ++u) {
      if (u < nc) {
        const long ko = (long)(cb + u) * 64;
        if (PRO == PRO_EMBED && ep) {
          xa[u] = *(const u32x4*)(ep + ko);
        } else if (xp) {
          xa[u] = *(const u32x4*)(xp + ko);
          xb[u] = *(const u32x4*)(xp + ko + 8);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < CW; ++u) {
      if (u < nc) {
        f16x8 fa = (f16x8){0, 0, 0, 0, 0, 0, 0, 0}, fb = fa;
        if (PRO == PRO_EMBED && ep) {
          i8x16_to_f16(xa[u], fa, fb);
          fa = fa * esc;
          fb = fb * esc;
        } else if (xp) {
          fa = __builtin_bit_cast(f16x8, xa[u]);
          fb = __builtin_bit_cast(f16x8, xb[u]);
          if (PRO == PRO_RMS) {
            const int k0 = (cb + u) * 64 + 16 * grp;
            const f16x8 wa = *(const f16x8*)(s_nw + k0);
            const f16x8 wb2 = *(const f16x8*)(s_nw + k0 + 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              fa[e] = (f16)((float)fa[e] * inv) * wa[e];
              fb[e] = (f16)((float)fb[e] * inv) * wb2[e];
            }
          }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          f16x8 wa, wbv;
          i8x16_to_f16(wr[u][t], wa, wbv);
          if (dense) {
            wa = wa * sw[t];
            wbv = wbv * sw[t];
          }
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wbv, fb, acc[t], 0, 0, 0);
        }
      }
    }
    cb += CW;
    nc = min(CW, c1 - cb);
#pragma unroll
    for (int u = 0; u < CW; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (u < nc) wr[u][t] = ldw<NTL>(wb[t] + (long)(cb + u) * 1024);
  }

  if constexpr (KW == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) gemv_epilogue<EPI>(a, n0, m0, t, lane, acc[t], epi_prefetch<EPI>(a, n0, m0, t, lane));
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
      gemv_epilogue<EPI>(a, n0, m0, t, l, s4, pre_e);
    }
  }
}

// LDS-staged variant: the block's x rows (after the prologue transform: RMSNorm or embedding
// gather) are built once in LDS by one wave per row at kernel start, while the first weight
// group is already in flight; the weight stream is then software-pipelined two groups deep and
// the MFMA B fragments come from LDS.  Used whenever the x tile fits in LDS.
constexpr int XPAD = 8;  // halfs of padding per LDS row (spreads rows over banks)

template <int NT, int KW, int PRO, int EPI, int CW, bool NTL>
__global__ __launch_bounds__(KW * 64) void gemv_xlds_kernel(const GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
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
  const int mv = min(16, M - m0);
  const int ldx = K + XPAD;
  f16* xs = (f16*)smem;

  const int8_t* wb[NT];
  f16 sw[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tile0 + t, ntiles - 1);
    wb[t] = a.wp + (long)tile * nch * 1024 + 16 * lane;
    sw[t] = dense ? a.s[min(n0 + 16 * t + row, N - 1)] : (f16)0.0f;
  }

  const bool epi_thread = (int)threadIdx.x < NT * 64;
  EpiPre pre_e;
  if (epi_thread) pre_e = epi_prefetch<EPI>(a, n0, m0, threadIdx.x >> 6, threadIdx.x & 63);

  u32x4 wA[CW][NT], wB[CW][NT];
  auto issue = [&](u32x4 (&w)[CW][NT], int cb) {
    const int nc = min(CW, c1 - cb);
#pragma unroll
    for (int u = 0; u < CW; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (u < nc) w[u][t] = ldw<NTL>(wb[t] + (long)(cb + u) * 1024);
  };
  if (c0 < c1) issue(wA, c0);

  // ---- stage x rows: wave w builds rows w, w + KW, ...
  for (int mr = wv; mr < mv; mr += KW) {
    const int m = m0 + mr;
    f16* dst = xs + (long)mr * ldx;
    if (PRO == PRO_EMBED) {
      const bool from_even = a.even && ((m & 1) == 0);
      const int b = a.even ? (m >> 1) : m;
      if (from_even) {
        const f16* src = a.even + (long)b * K;
        for (int k = lane * 8; k < K; k += 512) *(f16x8*)(dst + k) = ld8(src + k);
      } else {
        const long t = a.tok[(long)b * a.tok_stride];
        const long r = t + (long)a.cb * a.vocab;
        const bool ok = t >= 0 && t < a.vocab && r < a.erows;
        if (a.etab16) {
          const f16* src = a.etab16 + (ok ? r : 0) * K;
          const f16x8 z = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
          for (int k = lane * 8; k < K; k += 512) *(f16x8*)(dst + k) = ok ? ld8(src + k) : z;
          continue;
        }
        const int8_t* src = a.etab + (ok ? r : 0) * K;
        const f16 sc = ok ? a.escale[r] : (f16)0.0f;
        for (int k = lane * 16; k < K; k += 1024) {
          f16x8 lo = (f16x8){0, 0, 0, 0, 0, 0, 0, 0}, hi = lo;
          if (ok) {
            i8x16_to_f16(*(const u32x4*)(src + k), lo, hi);
            lo = lo * sc;
            hi = hi * sc;
          }
          *(f16x8*)(dst + k) = lo;
          *(f16x8*)(dst + k + 8) = hi;
        }
      }
    } else if (PRO == PRO_RMS) {
      // K <= NW_MAX: the whole row stays in registers (8 halfs per lane per 512)
      // the norm weights are loaded together with the row (one memory round trip, not two)
      const f16* src = a.x + (long)m * a.ldx;
      f16x8 v[NW_MAX / 512], nwv[NW_MAX / 512];
#pragma unroll
      for (int i = 0; i < NW_MAX / 512; ++i) {
        const int k = lane * 8 + 512 * i;
        if (k < K) {
          v[i] = ld8(src + k);
          nwv[i] = ld8(a.nw + k);
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NW_MAX / 512; ++i) {
        const int k = lane * 8 + 512 * i;
        if (k < K) {
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += (float)v[i][e] * (float)v[i][e];
        }
      }
      ss = wave_sum(ss);
      const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
      for (int i = 0; i < NW_MAX / 512; ++i) {
        const int k = lane * 8 + 512 * i;
        if (k < K) {
          f16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (f16)((float)v[i][e] * inv) * nwv[i][e];
          *(f16x8*)(dst + k) = o;
        }
      }
    } else {
      const f16* src = a.x + (long)m * a.ldx;
      for (int k = lane * 8; k < K; k += 512) *(f16x8*)(dst + k) = ld8(src + k);
    }
  }
  __syncthreads();

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const bool mval = row < mv;
  const f16* xrow = xs + (long)row * ldx + 16 * grp;

  auto compute = [&](const u32x4 (&w)[CW][NT], int cb) {
    const int nc = min(CW, c1 - cb);
#pragma unroll
    for (int u = 0; u < CW; ++u) {
      if (u < nc) {
        f16x8 fa = (f16x8){0, 0, 0, 0, 0, 0, 0, 0}, fb = fa;
        if (mval) {
          fa = *(const f16x8*)(xrow + (cb + u) * 64);
          fb = *(const f16x8*)(xrow + (cb + u) * 64 + 8);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          f16x8 wa, wbv;
          i8x16_to_f16(w[u][t], wa, wbv);
          if (dense) {
            wa = wa * sw[t];
            wbv = wbv * sw[t];
          }
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wbv, fb, acc[t], 0, 0, 0);
        }
      }
    }
  };

  for (int cb = c0; cb < c1;) {
    int nb = cb + CW;
    if (nb < c1) issue(wB, nb);
    compute(wA, cb);
    if (nb >= c1) break;
    cb = nb;
    nb = cb + CW;
    if (nb < c1) issue(wA, nb);
    compute(wB, cb);
    cb = nb;
  }

  // ---- cross-wave reduction (LDS reused after the x tile is dead) and epilogue
  __syncthreads();
  f32x4* red = (f32x4*)smem;  // [KW][NT][64]
#pragma unroll
  for (int t = 0; t < NT; ++t) red[(wv * NT + t) * 64 + lane] = acc[t];
  __syncthreads();
  for (int idx = threadIdx.x; idx < NT * 64; idx += KW * 64) {
    const int t = idx >> 6, l = idx & 63;
    f32x4 s4 = red[t * 64 + l];
#pragma unroll
    for (int v = 1; v < KW; ++v) s4 += red[(v * NT + t) * 64 + l];
    gemv_epilogue<EPI>(a, n0, m0, t, l, s4, pre_e);
  }
}

// Register-x variant: every wave loads, at kernel start, its own K-range of x (the B fragments
// of chunks [c0, c1), straight from memory in MFMA lane order) and then the first LA chunks of
// its weights; chunk u + LA is issued as chunk u is consumed.  No LDS tile or barrier sits
// before the MFMAs.  PRO_RMS needs the full-row statistics: each wave reduces the sum of
// squares over its own slice, one barrier exchanges the KW partial sums, and the norm weights
// are staged in LDS meanwhile.  MAXC >= c1 - c0 bounds the chunks a wave holds (host-checked).
template <int NT, int KW, int PRO, int EPI, bool NTL, int MAXC, int LA>
__global__ __launch_bounds__(KW * 64) void gemv_xreg_kernel(const GemvArgs a) {
  static_assert(PRO == PRO_PLAIN || PRO == PRO_RMS, "register-x prologue: plain or RMS");
  static_assert(KW * 512 >= NW_MAX, "one norm-weight vector per thread stages K <= NW_MAX");
  extern __shared__ __align__(16) unsigned char smem[];
  f32x4* red = (f32x4*)smem;                               // [KW][NT][64]
  float* s_ss = (float*)(smem + KW * NT * 64 * 16);        // [KW][16]
  f16* s_nw = (f16*)(smem + KW * NT * 64 * 16 + KW * 64);  // [K]
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
  // K-split (EPI_PARTIAL): block z covers chunks [z nchs, (z + 1) nchs); host: nch % ks == 0
  const int nchs = EPI == EPI_PARTIAL ? nch / a.ks : nch;
  const int c0 = (EPI == EPI_PARTIAL ? (int)blockIdx.z * nchs : 0) + (nchs * wv) / KW;
  const int nc = (nchs * (wv + 1)) / KW - (nchs * wv) / KW;
  const bool dense = a.dense != 0;

  // Issue order matters: loads complete in order for the wait counters, so the norm weights
  // and x (needed first) go out before the weights, and the weights go out chunk by chunk (the
  // MFMAs of chunk u wait only for chunks <= u).
  f16x8 nwt;
  const int kn = threadIdx.x * 8;
  if (PRO == PRO_RMS && kn < K) nwt = ld8(a.nw + kn);
  const bool mval = m0 + row < M;
  const f16* xp = a.x + (long)(mval ? m0 + row : 0) * a.ldx + (long)c0 * 64 + 16 * grp;
  f16x8 xa[MAXC], xb[MAXC];
#pragma unroll
  for (int u = 0; u < MAXC; ++u) {
    if (u < nc) {
      if (mval) {
        xa[u] = ld8(xp + u * 64);
        xb[u] = ld8(xp + u * 64 + 8);
      } else {
        xa[u] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
        xb[u] = xa[u];
      }
    }
  }

  u32x4 w[MAXC][NT];
  f16 sw[NT];
  const int8_t* wb = a.wp + (long)c0 * 1024 + 16 * lane;
  int tl[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) tl[t] = min(tile0 + t, ntiles - 1);
  // weight chunks [0, LA) now; chunk u + LA is issued when chunk u is consumed (at most LA
  // chunks of NT tiles in flight per wave)
#pragma unroll
  for (int u = 0; u < (LA < MAXC ? LA : MAXC); ++u)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (u < nc) w[u][t] = ldw<NTL>(wb + ((long)tl[t] * nch + u) * 1024);

  const bool epi_thread = (int)threadIdx.x < NT * 64;
  EpiPre pre_e;
  if (epi_thread) pre_e = epi_prefetch<EPI>(a, n0, m0, threadIdx.x >> 6, threadIdx.x & 63);
#pragma unroll
  for (int t = 0; t < NT; ++t) sw[t] = dense ? a.s[min(n0 + 16 * t + row, N - 1)] : (f16)0.0f;

  if (PRO == PRO_RMS) {
    if (kn < K) *(f16x8*)(s_nw + kn) = nwt;
    // sum of squares with v_dot2_f32_f16 (exact f16 products, fp32 sums): no fp32 copy of the
    // fragments stays live across the barrier below
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < MAXC; ++u)
      if (u < nc)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const f16x2 pa = (f16x2){xa[u][e], xa[u][e + 1]};
          const f16x2 pb = (f16x2){xb[u][e], xb[u][e + 1]};
          ss = __builtin_amdgcn_fdot2(pa, pa, ss, false);
          ss = __builtin_amdgcn_fdot2(pb, pb, ss, false);
        }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (grp == 0) s_ss[wv * 16 + row] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int v = 0; v < KW; ++v) tot += s_ss[v * 16 + row];
    const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
      if (u < nc) {
        const int k0 = (c0 + u) * 64 + 16 * grp;
        const f16x8 na = *(const f16x8*)(s_nw + k0);
        const f16x8 nb = *(const f16x8*)(s_nw + k0 + 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xa[u][e] = (f16)((float)xa[u][e] * inv) * na[e];
          xb[u][e] = (f16)((float)xb[u][e] * inv) * nb[e];
        }
      }
    }
  }

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < MAXC; ++u) {
    if (u < nc) {
      if (u + LA < MAXC && u + LA < nc) {
#pragma unroll
        for (int t = 0; t < NT; ++t) w[u + LA][t] = ldw<NTL>(wb + ((long)tl[t] * nch + u + LA) * 1024);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f16x8 wa, wbv;
        i8x16_to_f16(w[u][t], wa, wbv);
        if (dense) {
          wa = wa * sw[t];
          wbv = wbv * sw[t];
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, xa[u], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wbv, xb[u], acc[t], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < NT; ++t) red[(wv * NT + t) * 64 + lane] = acc[t];
  __syncthreads();
  for (int idx = threadIdx.x; idx < NT * 64; idx += KW * 64) {
    const int t = idx >> 6, l = idx & 63;
    f32x4 s4 = red[t * 64 + l];
#pragma unroll
    for (int v = 1; v < KW; ++v) s4 += red[(v * NT + t) * 64 + l];
    gemv_epilogue<EPI>(a, n0, m0, t, l, s4, pre_e);
  }
}

// Chunks per wave the register-x kernel can hold for NT tiles with KW waves per block (x and
// weight fragments stay within the per-lane register budget of KW waves per CU), 0 if none.
constexpr int xreg_maxc(int NT, int KW, int PRO) {
  return KW == 16 ? (NT == 1 ? 8 : NT == 2 ? 4 : 2) : (NT <= 2 || PRO == PRO_PLAIN ? 8 : 6);
}

template <int NT, int KW, int PRO, int EPI, bool NTL, int MAXC>
static int launch_xreg_one(const GemvArgs& a, hipStream_t st) {
  const int ntiles = (a.N + 15) / 16;
  dim3 grid((ntiles + NT - 1) / NT, (a.M + 15) / 16, EPI == EPI_PARTIAL ? a.ks : 1);
  const unsigned lds = KW * NT * 64 * 16 + KW * 64 + (PRO == PRO_RMS ? a.K * 2 : 0);
  // weight chunks in flight per wave: 16 KB (NT = 4 reads four tiles per chunk)
  constexpr int LA = NT >= 4 ? 4 : 16;
  hipLaunchKernelGGL((gemv_xreg_kernel<NT, KW, PRO, EPI, NTL, MAXC, LA>), grid, dim3(KW * 64), lds,
                     st, a);
  return ecd_launch_status();
}

// Launches the register-x kernel if the shape fits it; returns 1 (not launched) otherwise.
template <int NT, int KW, int PRO, int EPI, bool NTL>
static int launch_xreg(const GemvArgs& a, hipStream_t st) {
  if constexpr (PRO == PRO_EMBED || (PRO == PRO_RMS && KW != 8)) {
    return 1;
  } else {
    const int nch = (a.K >> 6) / (EPI == EPI_PARTIAL ? a.ks : 1);
    const int cpw = (nch + KW - 1) / KW;
    // Measured on every frame shape (MI355X): register x wins for the plain prologue at every
    // K and for the RMS prologue with 8 waves and at most two chunks per wave (K <= 1024); the
    // LDS tile wins for the RMS prologue over wider rows, whose partial-sum barrier waits for
    // every wave's slice of x.
    if (PRO == PRO_RMS && (a.K > NW_MAX || cpw > 2)) return 1;
    constexpr int MC = PRO == PRO_RMS ? 2 : xreg_maxc(NT, KW, PRO);
    if (cpw <= 1) return launch_xreg_one<NT, KW, PRO, EPI, NTL, 1>(a, st);
    if (cpw <= 2) return launch_xreg_one<NT, KW, PRO, EPI, NTL, 2>(a, st);
    if constexpr (MC >= 4) {
      if (cpw <= 4) return launch_xreg_one<NT, KW, PRO, EPI, NTL, 4>(a, st);
    }
    if constexpr (MC == 6) {
      if (cpw <= 6) return launch_xreg_one<NT, KW, PRO, EPI, NTL, 6>(a, st);
    }
    if constexpr (MC >= 8) {
      if (cpw <= 8) return launch_xreg_one<NT, KW, PRO, EPI, NTL, 8>(a, st);
    }
    return 1;
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

// Tile rule from a sweep of (tiles per block, waves per block, chunk group) over every frame
// shape on MI355X: 16 waves splitting K with 2-chunk load groups always wins; more 16-row tiles
// per block cut the re-read of x from L2 once there are enough tiles to keep 256 CUs busy.
static Cfg pick(int N, int K) {
  const int ntiles = (N + 15) / 16;
  (void)K;
  Cfg c{1, 16};
  if (ntiles >= 512) c = Cfg{4, 8};
  else if (ntiles >= 320) c.nt = 2;
  return c;
}

// Plain prologue (x straight from memory): from 512 tiles on, 2 tiles per workgroup of 16 waves
// (one workgroup per CU at 8192 columns) streams faster than 4 tiles on 8 waves, whose grid
// leaves half the CUs idle (8192 x 3072 at 1-8 rows, rotated weight sets: 9.8 -> 6.8 us).  The
// fused prologues keep pick: RMS over 1024 columns needs 8 waves for its register-x kernel.
static Cfg pick_plain(int N, int K) {
  Cfg c = pick(N, K);
  if ((N + 15) / 16 >= 512) c = Cfg{2, 16};
  return c;
}

// RMS prologue with a plain store (the codebook heads: 8197 columns, 513 tiles): from 512 to 767
// tiles, 3 tiles per workgroup, so that the busiest CU streams 3 tiles instead of 4 (171
// workgroups instead of 129; two per CU for some would double their share).
static Cfg pick_rms(int N, int K) {
  Cfg c = pick(N, K);
  const int ntiles = (N + 15) / 16;
  if (ntiles >= 512 && ntiles < 768) c.nt = 3;
  return c;
}

constexpr int LDS_MAX = 160 * 1024;

template <int NT, int KW, int PRO, int EPI, bool NTL>
static int launch_one(const GemvArgs& a, hipStream_t st) {
  {
    const int rc = launch_xreg<NT, KW, PRO, EPI, NTL>(a, st);
    if (rc != 1) return rc;
  }
  const int ntiles = (a.N + 15) / 16;
  dim3 grid((ntiles + NT - 1) / NT, (a.M + 15) / 16);
  const long xbytes = (long)min(16, a.M) * (a.K + XPAD) * 2;
  const long rbytes = (long)KW * NT * 64 * 16;
  const long lds = xbytes > rbytes ? xbytes : rbytes;
  if (lds <= LDS_MAX && (PRO != PRO_RMS || a.K <= NW_MAX)) {
    static bool attr = false;  // raise the dynamic LDS limit once per instantiation
    if (!attr) {
      const hipError_t e = hipFuncSetAttribute((const void*)gemv_xlds_kernel<NT, KW, PRO, EPI, 2, NTL>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, LDS_MAX);
      if (e != hipSuccess) return (int)e;
      attr = true;
    }
    hipLaunchKernelGGL((gemv_xlds_kernel<NT, KW, PRO, EPI, 2, NTL>), grid, dim3(KW * 64),
                       (unsigned)lds, st, a);
  } else {
    hipLaunchKernelGGL((gemv_fused_kernel<NT, KW, PRO, EPI, 2, NTL>), grid, dim3(KW * 64), 0, st, a);
  }
  return ecd_launch_status();
}

template <int PRO, int EPI, bool NTL>
static int launch_ntl(const GemvArgs& a, Cfg c, hipStream_t st) {
#define ECD_FCASE(NT_, KW_) \
  if (c.nt == NT_ && c.kw == KW_) return launch_one<NT_, KW_, PRO, EPI, NTL>(a, st);
  ECD_FCASE(1, 8)
  ECD_FCASE(1, 16)
  ECD_FCASE(2, 8)
  ECD_FCASE(2, 16)
  ECD_FCASE(3, 8)
  ECD_FCASE(4, 8)
  ECD_FCASE(4, 16)
#undef ECD_FCASE
  return ECD_ENOTSUP;
}

template <int PRO, int EPI>
static int launch(const GemvArgs& a, Cfg c, hipStream_t st) {
  if (PRO == PRO_RMS && a.K > NW_MAX) return ECD_ENOTSUP;
  return a.stream_hint ? launch_ntl<PRO, EPI, true>(a, c, st) : launch_ntl<PRO, EPI, false>(a, c, st);
}

// y[m, n] = fp16(sum_z ws[z][m][n] * s[n]) (dense: fp16(sum_z ws)), then + res as an fp16 add
// (the EPI_STORE numerics of the unsplit GEMV, with the K sum formed split by split in order).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int ks,
                                                            const f16* __restrict__ s,
                                                            const f16* __restrict__ res, long ldr,
                                                            f16* __restrict__ y, long ldy, int M,
                                                            int N, int dense) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * N) return;
  const int m = (int)(i / N), n = (int)(i - (long)m * N);
  float acc = 0.f;
  for (int z = 0; z < ks; ++z) acc += ws[(long)z * M * N + i];
  f16 o = (f16)(dense ? acc : acc * (float)s[n]);
  if (res) o = o + res[(long)m * ldr + n];
  y[(long)m * ldy + n] = o;
}

template <bool NTL>
static int launch_splitk(const GemvArgs& a, Cfg c, hipStream_t st) {
  int rc = 1;
#define ECD_SK(NT_, KW_) \
  if (c.nt == NT_ && c.kw == KW_) rc = launch_xreg<NT_, KW_, PRO_PLAIN, EPI_PARTIAL, NTL>(a, st);
  ECD_SK(1, 16)
  ECD_SK(2, 16)
  ECD_SK(4, 8)
#undef ECD_SK
  if (rc == 1) return ECD_ENOTSUP;
  if (rc != ECD_OK) return rc;
  const long n = (long)a.M * a.N;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     a.ws, a.ks, a.s, a.res, a.ldr, a.y, a.ldy, a.M, a.N, a.dense);
  return ecd_launch_status();
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
                 void* y, long ldy, int M, int N, int K, int flags, int nt, int kw, void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.wp = (const int8_t*)wp; a.s = (const f16*)s;
  a.M = M; a.N = N; a.K = K; a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1;
  a.res = (const f16*)res; a.ldr = ldr; a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !x || !y || ldx < K || (ldx % 8) || !aligned16(x) || ldy < N ||
      (res && ldr < N))
    return ECD_EINVAL;
  Cfg c = pick_plain(N, K);
  if (nt > 0) c.nt = nt;
  if (kw > 0) c.kw = kw;
  return launch<PRO_PLAIN, EPI_STORE>(a, c, (hipStream_t)stream);
}

int ecd_gemv_i8p_splitk(const void* x, long ldx, const void* wp, const void* s, const void* res,
                        long ldr, void* y, long ldy, int M, int N, int K, int ks, float* ws,
                        int flags, void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.wp = (const int8_t*)wp; a.s = (const f16*)s;
  a.M = M; a.N = N; a.K = K; a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1;
  a.res = (const f16*)res; a.ldr = ldr; a.y = (f16*)y; a.ldy = ldy; a.ws = ws; a.ks = ks;
  if (check_common(a) || !x || !y || !ws || ldx < K || (ldx % 8) || !aligned16(x) || ldy < N ||
      (res && ldr < N) || ks < 1 || ((K / 64) % ks))
    return ECD_EINVAL;
  const Cfg c = pick(N, K);
  return a.stream_hint ? launch_splitk<true>(a, c, (hipStream_t)stream)
                       : launch_splitk<false>(a, c, (hipStream_t)stream);
}

int ecd_rms_gemv_i8p(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* y, long ldy, int M, int N, int K, int flags,
                     void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.N = N; a.K = K; a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1;
  a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !x || !nw || !y || ldx < K || (ldx % 8) || !aligned16(x) ||
      !aligned16(nw) || ldy < N)
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_STORE>(a, pick_rms(N, K), (hipStream_t)stream);
}

int ecd_rms_qkv_rope(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, const float* rope, const int64_t* pos, void* q, void* kc,
                     void* vc, int M, int S, int Hq, int Hk, int L, int HD, int K, int flags,
                     void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.K = K; a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1;
  a.N = (Hq + 2 * Hk) * HD;
  a.rope = rope; a.pos = pos; a.q = (f16*)q; a.kc = (f16*)kc; a.vc = (f16*)vc;
  a.S = S; a.Hq = Hq; a.Hk = Hk; a.L = L; a.HD = HD; a.qrows = (flags >> 2) & 1;
  if (check_common(a) || !x || !nw || !rope || !pos || !q || (!a.qrows && (!kc || !vc)) ||
      S <= 0 || Hq <= 0 ||
      Hk <= 0 || L <= 0 || HD <= 0 || (HD % 4) || (Hq % Hk) || ldx < K || (ldx % 8) ||
      !aligned16(x) || !aligned16(nw))
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_ROPE>(a, pick(a.N, K), (hipStream_t)stream);
}

int ecd_rms_w13_silu(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* mm, int M, int F, int K, int flags, void* stream) {
  GemvArgs a = {};
  a.x = (const f16*)x; a.ldx = ldx; a.nw = (const f16*)nw; a.eps = eps;
  a.wp = (const int8_t*)wp; a.s = (const f16*)s; a.M = M; a.N = 2 * F; a.K = K;
  a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1; a.mm = (f16*)mm;
  if (check_common(a) || !x || !nw || !mm || F <= 0 || (F % 2) || ldx < K || (ldx % 8) ||
      !aligned16(x) || !aligned16(nw))
    return ECD_EINVAL;
  return launch<PRO_RMS, EPI_SILU>(a, pick(a.N, K), (hipStream_t)stream);
}

int ecd_embed_gemv_i8p(const int64_t* tok, long tok_stride, const void* table, const void* tscale,
                       long trows, int cb, int vocab, const void* even, const void* wp,
                       const void* s, void* y, long ldy, int M, int N, int K, int flags,
                       void* stream) {
  GemvArgs a = {};
  a.tok = tok; a.tok_stride = tok_stride; a.erows = trows; a.cb = cb; a.vocab = vocab;
  if (tscale) {
    a.etab = (const int8_t*)table;
    a.escale = (const f16*)tscale;
  } else {
    a.etab16 = (const f16*)table;
  }
  a.even = (const f16*)even; a.wp = (const int8_t*)wp; a.s = (const f16*)s;
  a.M = M; a.N = N; a.K = K; a.dense = flags & 1; a.stream_hint = (flags >> 1) & 1; a.y = (f16*)y; a.ldy = ldy;
  if (check_common(a) || !tok || !table || !y || tok_stride <= 0 || trows <= 0 ||
      cb < 0 || vocab <= 0 || ldy < N || !aligned16(table) || (even && !aligned16(even)) ||
      (even && (M & 1)))
    return ECD_EINVAL;
  return launch<PRO_EMBED, EPI_STORE>(a, pick(N, K), (hipStream_t)stream);
}

}  // extern "C"
