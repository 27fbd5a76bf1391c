// Prompt-pass GEMM on packed int8 weights (gfx950 MFMA), the reference's dense numerics for
// many rows (app/kernels.py:46-49: dequantise, then GEMM):
//   y[m, n] = fp16( sum_k x[m, k] * fp16(q[n, k] * s[n]) )      fp32 accumulation
//   EPI_STORE: y (+ res as an fp16 add);  EPI_SILU: rows interleaved (w1 row j at 2j, w3 row j
//   at 2j + 1), mm[m, j] = fp16(fp16(silu(y[m, 2j])) * y[m, 2j + 1]) (app/kernels.py:171-180).
//
// Weights use the lane-ordered packed layout of gemv_fused.hip: chunk (tile, c) = 16 rows x
// 64 bytes stored so that lane l's 16 bytes are row l & 15, k = 64c + 16 (l >> 4) .. +15.
//
// Tiling: a block computes 128 output features x 128 rows with 4 waves; wave (wn, wm) owns
// 64 features x 64 rows = 4 x 4 tiles of v_mfma_f32_16x16x32_f16 (weights = A operand, x = B
// operand).  K advances in 64-wide chunks staged through LDS (weights as packed 1 KB tiles,
// x rows padded to 72 halfs so the B-fragment reads spread over the banks), double-buffered:
// the next chunk's global loads are in flight while the current one is multiplied.  Each
// 16-byte weight fragment is dequantised once and used by 4 row tiles; each x fragment is
// used by 4 feature tiles.
//
// Block order is XCD-aware: the row blocks that share a weight tile get block ids that are
// equal modulo 8, so they run on one XCD and re-read the tile from its L2.
#include "common.h"

namespace ecd {

enum { GEPI_STORE = 0, GEPI_SILU = 1 };

constexpr int GT_N = 128;   // output features per block
constexpr int GT_M = 128;   // rows per block
constexpr int GXS = 72;     // LDS row stride of the x tile, halfs (64 + 8 padding)

template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8p_kernel(
    const f16* __restrict__ x, long ldx, const int8_t* __restrict__ wp,
    const f16* __restrict__ s, const f16* __restrict__ res, long ldr, f16* __restrict__ y,
    long ldy, int M, int N, int K, int nfb, int nmb) {
  __shared__ __align__(16) int8_t lw[2][8 * 1024];
  __shared__ __align__(16) f16 lx[2][GT_M * GXS];

  // XCD-aware block order: blocks b and b + 8 run on the same XCD.  Feature block fb and row
  // block mb map to b = (fb / 8) * (8 * nmb) + mb * 8 + fb % 8.
  const int b = blockIdx.x;
  const int grp8 = b / (8 * nmb);
  const int rem = b - grp8 * 8 * nmb;
  const int mb = rem >> 3;
  const int fb = grp8 * 8 + (rem & 7);
  if (fb >= nfb) return;  // padding blocks of the last group of 8 (uniform per block)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int wn = wv & 1, wm = wv >> 1;
  const int n0 = fb * GT_N;
  const int m0 = mb * GT_M;
  const int nch = K >> 6;
  const int ntiles = (N + 15) >> 4;

  // global -> register staging of one chunk: weights (8 tiles x 1 KB, 32 bytes per thread),
  // x (128 rows x 128 bytes, 64 bytes per thread)
  const int wt = tid >> 5;                       // tile of this thread's weight bytes
  const int wo = (tid & 31) * 32;                // byte offset inside the tile's 1 KB chunk
  const int wtile = min(n0 / 16 + wt, ntiles - 1);
  const int8_t* wsrc = wp + (long)wtile * nch * 1024 + wo;
  const int xr = tid >> 1;                       // x row of this thread (0..127)
  const int xo = (tid & 1) * 32;                 // first half of the row's 64-k chunk
  const bool xok = m0 + xr < M;
  const f16* xsrc = x + (long)(xok ? m0 + xr : 0) * ldx + xo;

  u32x4 rw[2], rx[4];
  auto gload = [&](int c) {
    rw[0] = *(const u32x4*)(wsrc + (long)c * 1024);
    rw[1] = *(const u32x4*)(wsrc + (long)c * 1024 + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      rx[i] = xok ? *(const u32x4*)(xsrc + (long)c * 64 + 8 * i) : (u32x4){0u, 0u, 0u, 0u};
  };
  auto lstore = [&](int buf) {
    *(u32x4*)(&lw[buf][wt * 1024 + wo]) = rw[0];
    *(u32x4*)(&lw[buf][wt * 1024 + wo + 16]) = rw[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) *(u32x4*)(&lx[buf][xr * GXS + xo + 8 * i]) = rx[i];
  };

  // per-lane dequantisation scales of the 4 feature tiles (row lane & 15 of each)
  f16 sc[4];
#pragma unroll
  for (int ft = 0; ft < 4; ++ft) sc[ft] = s[min(n0 + (wn * 4 + ft) * 16 + (lane & 15), N - 1)];

  f32x4 acc[4][4];
#pragma unroll
  for (int ft = 0; ft < 4; ++ft)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[ft][rt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    if (c + 1 < nch) gload(c + 1);
    f16x8 wa[4], wb[4];
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      const u32x4 raw = *(const u32x4*)(&lw[buf][(wn * 4 + ft) * 1024 + 16 * lane]);
      i8x16_to_f16(raw, wa[ft], wb[ft]);
      wa[ft] = wa[ft] * sc[ft];
      wb[ft] = wb[ft] * sc[ft];
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const f16* xp = &lx[buf][(wm * 64 + rt * 16 + (lane & 15)) * GXS + 16 * (lane >> 4)];
      const f16x8 fa = *(const f16x8*)xp;
      const f16x8 fb2 = *(const f16x8*)(xp + 8);
#pragma unroll
      for (int ft = 0; ft < 4; ++ft) {
        acc[ft][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[ft], fa, acc[ft][rt], 0, 0, 0);
        acc[ft][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[ft], fb2, acc[ft][rt], 0, 0, 0);
      }
    }
    if (c + 1 < nch) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds features nb + r (r < 4) of row m for every (ft, rt)
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int m = m0 + wm * 64 + rt * 16 + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      const int nb = n0 + (wn * 4 + ft) * 16 + 4 * (lane >> 4);
      if (nb >= N) continue;
      f16 yv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) yv[r] = (f16)acc[ft][rt][r];
      if (EPI == GEPI_STORE) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (nb + r < N) {
            f16 o = yv[r];
            if (res) o = o + res[(long)m * ldr + nb + r];
            y[(long)m * ldy + nb + r] = o;
          }
        }
      } else {  // (a_j, b_j, a_j+1, b_j+1) with j = nb / 2; N even
        const int j = nb >> 1;
        const float a0 = (float)yv[0], a1 = (float)yv[2];
        f16x2 o;
        o.x = (f16)(a0 / (1.0f + expf(-a0))) * yv[1];
        o.y = (f16)(a1 / (1.0f + expf(-a1))) * yv[3];
        *(f16x2*)(y + (long)m * ldy + j) = o;
      }
    }
  }
}

template <int EPI>
static int launch_gemm(const f16* x, long ldx, const int8_t* wp, const f16* s, const f16* res,
                       long ldr, f16* y, long ldy, int M, int N, int K, hipStream_t st) {
  const int nfb = (N + GT_N - 1) / GT_N;
  const int nmb = (M + GT_M - 1) / GT_M;
  const long blocks = (long)((nfb + 7) / 8) * 8 * nmb;
  if (blocks > 0x7FFFFFFFL) return ECD_ENOTSUP;
  hipLaunchKernelGGL((gemm_i8p_kernel<EPI>), dim3((unsigned)blocks), dim3(256), 0, st, x, ldx, wp,
                     s, res, ldr, y, ldy, M, N, K, nfb, nmb);
  return ecd_launch_status();
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace ecd

using namespace ecd;

extern "C" {

int ecd_gemm_i8p(const void* x, long ldx, const void* wp, const void* s, const void* res,
                 long ldr, void* y, long ldy, int M, int N, int K, void* stream) {
  if (!x || !wp || !s || !y || M <= 0 || N <= 0 || K <= 0 || (K % 64) || ldx < K || (ldx % 8) ||
      !al16(x) || !al16(wp) || ldy < N || (res && ldr < N))
    return ECD_EINVAL;
  return launch_gemm<GEPI_STORE>((const f16*)x, ldx, (const int8_t*)wp, (const f16*)s,
                                 (const f16*)res, ldr, (f16*)y, ldy, M, N, K,
                                 (hipStream_t)stream);
}

int ecd_gemm_i8p_silu(const void* x, long ldx, const void* wp, const void* s, void* mm,
                      long ldm, int M, int F, int K, void* stream) {
  if (!x || !wp || !s || !mm || M <= 0 || F <= 0 || (F % 2) || K <= 0 || (K % 64) || ldx < K ||
      (ldx % 8) || !al16(x) || !al16(wp) || ldm < F || (ldm % 2) || ((uintptr_t)mm & 3))
    return ECD_EINVAL;
  return launch_gemm<GEPI_SILU>((const f16*)x, ldx, (const int8_t*)wp, (const f16*)s, nullptr, 0,
                                (f16*)mm, ldm, M, 2 * F, K, (hipStream_t)stream);
}

}  // extern "C"
