// int8 per-output-channel weight x fp16 activation GEMV / skinny GEMM for gfx950.
//
// Computes, for x [M, K] fp16, q [N, K] int8 (K contiguous), s [N] fp16:
//   GEMV numerics  (M <= 16, reference app/kernels.py:20-37):
//       y[m, n] = fp16( fp32(s[n]) * sum_k x[m,k] * q[n,k] )      (fp32 accumulation)
//   dense numerics (M > 16, reference app/kernels.py:46-49, dequantise then GEMM):
//       y[m, n] = fp16( sum_k x[m,k] * fp16(fp16(q[n,k]) * s[n]) )
//   then, with a residual, y = fp16(y + res[m, n])  (app/kernels.py:35-36, :48).
//
// Design (HBM streaming; the weights are read exactly once per 16-row M tile):
//   * one MFMA tile is 16 output channels (n) x 16 batch rows (m); the weights are the
//     A operand, so lane l owns weight row n0 + (l & 15) and loads 16 contiguous bytes
//     of it at k-offset 16 * (l >> 4) of each 64-wide k chunk: one global_load_dwordx4 per
//     lane covers 16 rows x 64 bytes.
//   * the 16 codes become two f16x8 operands in registers (exact int8 -> f16), feeding two
//     v_mfma_f32_16x16x32_f16; the x fragment (B operand) holds the same 16 k for batch row
//     m0 + (l & 15) (zero for rows >= M).  The k order inside an MFMA is a free permutation
//     as long as A and B agree, which they do by construction.
//   * a block holds KW waves that split the k chunks; partial 16x16 tiles are reduced
//     through LDS in a fixed order (deterministic), then scaled, rounded and stored.
#include "common.h"

namespace ecd {

template <int NT, int KW, int U, bool RES, bool DENSE>
__global__ __launch_bounds__(KW * 64) void gemv_i8_kernel(
    const f16* __restrict__ x, long ldx, const int8_t* __restrict__ w, const f16* __restrict__ s,
    const f16* __restrict__ res, long ldr, f16* __restrict__ y, long ldy, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int n0 = blockIdx.x * (16 * NT);
  const int m0 = blockIdx.y * 16;

  const int nch = K >> 6;
  const int c0 = (nch * wv) / KW;
  const int c1 = (nch * (wv + 1)) / KW;

  const int8_t* wp[NT];
  f16 sw[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = min(n0 + 16 * t + row, N - 1);
    wp[t] = w + (long)n * K + 16 * grp;
    sw[t] = DENSE ? s[n] : (f16)0.0f;
  }
  const bool mval = (m0 + row) < M;
  const f16* xp = x + (long)(mval ? m0 + row : 0) * ldx + 16 * grp;

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto step = [&](const u32x4 (&wr)[NT], const u32x4& xa, const u32x4& xb) {
    const f16x8 fa = __builtin_bit_cast(f16x8, xa);
    const f16x8 fb = __builtin_bit_cast(f16x8, xb);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f16x8 wa, wb;
      i8x16_to_f16(wr[t], wa, wb);
      if (DENSE) {
        wa = wa * sw[t];
        wb = wb * sw[t];
      }
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, fb, acc[t], 0, 0, 0);
    }
  };

  int c = c0;
  for (; c + U <= c1; c += U) {
    u32x4 wr[U][NT];
    u32x4 xr[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wr[u][t] = __builtin_nontemporal_load((const u32x4*)(wp[t] + (long)(c + u) * 64));
      if (mval) {
        xr[u][0] = *(const u32x4*)(xp + (long)(c + u) * 64);
        xr[u][1] = *(const u32x4*)(xp + (long)(c + u) * 64 + 8);
      } else {
        xr[u][0] = (u32x4){0u, 0u, 0u, 0u};
        xr[u][1] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) step(wr[u], xr[u][0], xr[u][1]);
  }
  for (; c < c1; ++c) {
    u32x4 wr[NT];
    u32x4 xa = (u32x4){0u, 0u, 0u, 0u}, xb = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wr[t] = __builtin_nontemporal_load((const u32x4*)(wp[t] + (long)c * 64));
    if (mval) {
      xa = *(const u32x4*)(xp + (long)c * 64);
      xb = *(const u32x4*)(xp + (long)c * 64 + 8);
    }
    step(wr, xa, xb);
  }

  auto epilogue = [&](int t, int l, const f32x4& a) {
    const int m = m0 + (l & 15);
    if (m >= M) return;
    const int nb = n0 + 16 * t + 4 * (l >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nb + r;
      if (n < N) {
        const float v = DENSE ? a[r] : a[r] * (float)s[n];
        f16 o = (f16)v;
        if (RES) o = o + res[(long)m * ldr + n];
        y[(long)m * ldy + n] = o;
      }
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
      f32x4 a = red[0][t][l];
#pragma unroll
      for (int v = 1; v < KW; ++v) a += red[v][t][l];
      epilogue(t, l, a);
    }
  }
}

// Any K, any alignment: one wave per output channel, lanes stride over k.
// Same numerics as the tiled kernel; used for shapes the tiled kernel does not cover.
template <bool RES, bool DENSE>
__global__ __launch_bounds__(256) void gemv_i8_generic_kernel(
    const f16* __restrict__ x, long ldx, const int8_t* __restrict__ w, const f16* __restrict__ s,
    const f16* __restrict__ res, long ldr, f16* __restrict__ y, long ldy, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int m0 = blockIdx.y * 16;
  if (n >= N) return;
  const int8_t* wr = w + (long)n * K;
  const f16 sn = s[n];
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  const int mt = min(16, M - m0);
  for (int k = lane; k < K; k += 64) {
    f16 wk = (f16)(float)wr[k];
    if (DENSE) wk = wk * sn;
    const float wf = (float)wk;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < mt) acc[i] += (float)x[(long)(m0 + i) * ldx + k] * wf;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == 0 && i < mt) {
      const int m = m0 + i;
      f16 o = (f16)(DENSE ? v : v * (float)sn);
      if (RES) o = o + res[(long)m * ldr + n];
      y[(long)m * ldy + n] = o;
    }
  }
}

struct GemvCfg {
  int nt, kw;
};

// Tile choice: enough waves to cover the 256 CUs several times while every wave still
// streams several 64-wide chunks per weight row.
static GemvCfg pick_cfg(int N, int K) {
  const int ntiles = (N + 15) / 16;
  const int nch = K / 64;
  int kw = 8;
  if (nch >= 128) kw = 16;
  if (nch < 16) kw = nch >= 4 ? 4 : 1;
  int nt = 1;
  if (ntiles >= 1024 && nch <= 48) nt = 2;
  return {nt, kw};
}

template <int NT, int KW, bool RES, bool DENSE>
static void launch_tiled(const f16* x, long ldx, const int8_t* w, const f16* s, const f16* res,
                         long ldr, f16* y, long ldy, int M, int N, int K, hipStream_t st) {
  dim3 grid((N + 16 * NT - 1) / (16 * NT), (M + 15) / 16);
  hipLaunchKernelGGL((gemv_i8_kernel<NT, KW, 4, RES, DENSE>), grid, dim3(KW * 64), 0, st, x, ldx,
                     w, s, res, ldr, y, ldy, M, N, K);
}

template <bool RES, bool DENSE>
static int dispatch(const GemvCfg& c, const f16* x, long ldx, const int8_t* w, const f16* s,
                    const f16* res, long ldr, f16* y, long ldy, int M, int N, int K,
                    hipStream_t st) {
#define ECD_GEMV_CASE(NT_, KW_)                                                        \
  if (c.nt == NT_ && c.kw == KW_) {                                                    \
    launch_tiled<NT_, KW_, RES, DENSE>(x, ldx, w, s, res, ldr, y, ldy, M, N, K, st);   \
    return ECD_OK;                                                                     \
  }
  ECD_GEMV_CASE(1, 1)
  ECD_GEMV_CASE(1, 4)
  ECD_GEMV_CASE(1, 8)
  ECD_GEMV_CASE(1, 16)
  ECD_GEMV_CASE(2, 1)
  ECD_GEMV_CASE(2, 4)
  ECD_GEMV_CASE(2, 8)
  ECD_GEMV_CASE(2, 16)
  ECD_GEMV_CASE(4, 4)
  ECD_GEMV_CASE(4, 8)
#undef ECD_GEMV_CASE
  return ECD_ENOTSUP;
}

}  // namespace ecd

using namespace ecd;

static int gemv_entry(const void* x, long ldx, const void* w, const void* s, const void* res,
                      long ldr, void* y, long ldy, int M, int N, int K, int dense, int nt, int kw,
                      void* stream) {
  if (!x || !w || !s || !y || M <= 0 || N <= 0 || K <= 0 || ldx < K || ldy < N ||
      (res && ldr < N))
    return ECD_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const f16* xh = (const f16*)x;
  const int8_t* wq = (const int8_t*)w;
  const f16* sh = (const f16*)s;
  const f16* rh = (const f16*)res;
  f16* yh = (f16*)y;
  const bool tiled = (K % 64 == 0) && (ldx % 8 == 0) && (((uintptr_t)x & 15) == 0) &&
                     (((uintptr_t)w & 15) == 0);
  int rc = ECD_OK;
  if (tiled) {
    GemvCfg c = pick_cfg(N, K);
    if (nt > 0) c.nt = nt;
    if (kw > 0) c.kw = kw;
    if (dense) {
      rc = res ? dispatch<true, true>(c, xh, ldx, wq, sh, rh, ldr, yh, ldy, M, N, K, st)
               : dispatch<false, true>(c, xh, ldx, wq, sh, rh, ldr, yh, ldy, M, N, K, st);
    } else {
      rc = res ? dispatch<true, false>(c, xh, ldx, wq, sh, rh, ldr, yh, ldy, M, N, K, st)
               : dispatch<false, false>(c, xh, ldx, wq, sh, rh, ldr, yh, ldy, M, N, K, st);
    }
    if (rc != ECD_OK) return rc;
  } else {
    dim3 grid((N + 3) / 4, (M + 15) / 16);
    if (dense) {
      if (res)
        hipLaunchKernelGGL((gemv_i8_generic_kernel<true, true>), grid, dim3(256), 0, st, xh, ldx,
                           wq, sh, rh, ldr, yh, ldy, M, N, K);
      else
        hipLaunchKernelGGL((gemv_i8_generic_kernel<false, true>), grid, dim3(256), 0, st, xh, ldx,
                           wq, sh, rh, ldr, yh, ldy, M, N, K);
    } else {
      if (res)
        hipLaunchKernelGGL((gemv_i8_generic_kernel<true, false>), grid, dim3(256), 0, st, xh,
                           ldx, wq, sh, rh, ldr, yh, ldy, M, N, K);
      else
        hipLaunchKernelGGL((gemv_i8_generic_kernel<false, false>), grid, dim3(256), 0, st, xh,
                           ldx, wq, sh, rh, ldr, yh, ldy, M, N, K);
    }
  }
  return ecd_launch_status();
}

extern "C" {

int ecd_gemv_i8(const void* x, long ldx, const void* w, const void* s, const void* res, long ldr,
                void* y, long ldy, int M, int N, int K, int dense, void* stream) {
  // many rows with the dense numerics (the reference's M > 16 path): the MFMA GEMM reads the
  // weights once per XCD instead of once per 16-row tile
  if (dense && M > 16 && x && w && s && y && N > 0 && K > 0 && ldx >= K && ldy >= N &&
      (!res || ldr >= N)) {
    const int rc = gemm_i8_rowmajor((const f16*)x, ldx, (const int8_t*)w, (const f16*)s,
                                    (const f16*)res, ldr, (f16*)y, ldy, M, N, K,
                                    (hipStream_t)stream);
    if (rc != 1) return rc;
  }
  return gemv_entry(x, ldx, w, s, res, ldr, y, ldy, M, N, K, dense, 0, 0, stream);
}

int ecd_gemv_i8_tuned(const void* x, long ldx, const void* w, const void* s, const void* res,
                      long ldr, void* y, long ldy, int M, int N, int K, int dense, int nt, int kw,
                      void* stream) {
  return gemv_entry(x, ldx, w, s, res, ldr, y, ldy, M, N, K, dense, nt, kw, stream);
}

}  // extern "C"
