// Prompt-pass GEMM on packed int8 weights (gfx950 MFMA), the reference's dense numerics for
// many rows (app/kernels.py:46-49: dequantise, then GEMM):
//   y[m, n] = fp16( sum_k x[m, k] * fp16(q[n, k] * s[n]) )      fp32 accumulation
//   EPI_STORE: y (+ res as an fp16 add);  EPI_SILU: rows interleaved (w1 row j at 2j, w3 row j
//   at 2j + 1), mm[m, j] = fp16(fp16(silu(y[m, 2j])) * y[m, 2j + 1]) (app/kernels.py:171-180);
//   EPI_ROPE: y is the q | k | v projection; the interleaved pairs of the q and k heads are
//   rotated by the RoPE table at the row's position and q goes to its buffer, k and v into the
//   cache slot (app/kernels.py:78-107: the same fp16 input, fp32 rotation and rounding as the
//   rope_kv kernel).
//
// Weights use the lane-ordered packed layout of gemv_fused.hip: chunk (tile, c) = 16 rows x
// 64 bytes stored so that lane l's 16 bytes are row l & 15, k = 64c + 16 (l >> 4) .. +15.  The
// row-major variant (RM) reads the same 16 bytes straight from an [N, K] int8 matrix (the
// layout int8_mm receives, app/kernels.py:40-49): the DMA lands them in LDS in the same lane
// order, so everything after the load is shared.
//
// Tiling: a block computes 128 output features x 128 rows with 4 waves; wave w owns features
// 32 w .. 32 w + 31 for all 128 rows = 2 x 8 tiles of v_mfma_f32_16x16x32_f16 (weights = A
// operand, x = B operand), so each weight fragment is dequantised by one wave only (the
// dequantisation is the kernel's largest VALU cost).  K advances in 64-wide chunks that go straight from global memory into two LDS
// stages (global_load_lds_dwordx4: each wave instruction writes 1 KB of LDS in lane order): the
// next chunk is in flight while one is multiplied, no registers stage the data, and 48 KB of
// LDS per block leave room for three blocks per CU.
// Weights arrive as packed 1 KB tiles; the 16-byte pieces of each x row (128 bytes per chunk)
// are XOR-swizzled by row (piece p of row r at position p ^ (r & 7)), which the loads produce
// by choosing each lane's source and which spreads the fragment reads over the banks.  Each
// 16-byte weight fragment is dequantised once and used by 8 row tiles; each x fragment is used
// by 2 feature tiles.
//
// The kernel orders the DMA itself: at the top of step c each thread waits for its own loads of
// chunk c (vmcnt 0), a barrier makes the chunk of every wave visible and frees the stage read
// in step c - 1, and only then are chunk c + 1's loads issued into that stage.
//
// Block order is XCD-aware: the row blocks that share a weight tile get block ids that are
// equal modulo 8, so they run on one XCD and re-read the tile from its L2.
#include "common.h"

namespace ecd {

enum { GEPI_STORE = 0, GEPI_SILU = 1, GEPI_ROPE = 2 };

// Operands of the RoPE + cache-write epilogue: row m is batch item m / S at position pos[m];
// rope [L, HD] fp32 holds (cos, sin) of pair i at columns 2i, 2i + 1.
struct RopeOut {
  const float* rope;
  const int64_t* pos;
  f16* q;   // [M, Hq * HD]
  f16* kc;  // [B, Hk, L, HD]
  f16* vc;
  int S, Hq, Hk, L, HD;
};

constexpr int GT_N = 128;   // output features per block
constexpr int GT_M = 128;   // rows per block
constexpr int GT_NS = 2;    // LDS stages

template <int EPI, bool RM>
__global__ __launch_bounds__(256) void gemm_i8p_kernel(
    const f16* __restrict__ x, long ldx, const int8_t* __restrict__ wp,
    const f16* __restrict__ s, const f16* __restrict__ res, long ldr, f16* __restrict__ y, long ldy, int M, int N, int K,
    int nfb, int nmb, RopeOut ro) {
  constexpr int WB = 1024;  // bytes of one (tile, chunk) of packed weights
  __shared__ __align__(16) int8_t lw[GT_NS][8 * WB];
  __shared__ __align__(16) f16 lx[GT_NS][GT_M * 64];

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
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = fb * GT_N;
  const int m0 = mb * GT_M;
  const int nch = K >> 6;
  const int ntiles = (N + 15) >> 4;

  // sources of this thread's loads: weight tiles wv and wv + 4 (16 bytes of each 1 KB chunk);
  // x rows 8 (4 wv + i) + (lane >> 3), swizzled piece (lane & 7) ^ (lane >> 3).  Rows past M
  // read row M - 1 and tiles past N the last tile (their results are never stored), so every
  // thread issues the same number of loads.
  // The addresses are a wave-uniform base (SGPRs, advanced per chunk by scalar adds) plus a
  // per-lane byte offset fixed for the whole loop (the host keeps the x buffer below 2 GiB).
  const int t0 = min(n0 / 16 + wv, ntiles - 1), t1 = min(n0 / 16 + 4 + wv, ntiles - 1);
  const int8_t* wbase0 = wp + (RM ? (long)t0 * 16 * K : (long)t0 * nch * WB);
  const int8_t* wbase1 = wp + (RM ? (long)t1 * 16 * K : (long)t1 * nch * WB);
  // row-major: row 16 t + (lane & 15) (the last row for rows past N), bytes 16 (lane >> 4) of
  // each 64-byte chunk; the per-lane offsets stay below 16 K bytes
  const uint32_t woff0 = RM ? (uint32_t)((min(16 * t0 + (lane & 15), N - 1) - 16 * t0) * K +
                                         16 * (lane >> 4))
                            : 16u * lane;
  const uint32_t woff1 = RM ? (uint32_t)((min(16 * t1 + (lane & 15), N - 1) - 16 * t1) * K +
                                         16 * (lane >> 4))
                            : 16u * lane;
  constexpr long WSTEP = RM ? 64 : WB;  // bytes between consecutive chunks of a tile
  const int xpiece = (lane & 7) ^ (lane >> 3);
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    xoff[i] = (uint32_t)((long)min(m0 + 8 * (4 * wv + i) + (lane >> 3), M - 1) * ldx * 2 +
                         16 * xpiece);
  auto issue = [&](int c, int st) {
    lds_dma16(wbase0 + (long)c * WSTEP, woff0, &lw[st][wv * WB]);
    lds_dma16(wbase1 + (long)c * WSTEP, woff1, &lw[st][(4 + wv) * WB]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lds_dma16(x + (long)c * 64, xoff[i], &lx[st][8 * (4 * wv + i) * 64]);
  };

  // per-lane dequantisation scales of the 2 feature tiles (row lane & 15 of each)
  f16 sc[2];
#pragma unroll
  for (int ft = 0; ft < 2; ++ft) sc[ft] = s[min(n0 + (wv * 2 + ft) * 16 + (lane & 15), N - 1)];

  f32x4 acc[2][8];
#pragma unroll
  for (int ft = 0; ft < 2; ++ft)
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) acc[ft][rt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  issue(0, 0);
  const int sw = lane & 7;  // swizzle of the rows this lane reads (row & 7 == lane & 7)
  for (int c = 0; c < nch; ++c) {
    wait_vm0();  // this thread's loads of chunk c have landed in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // chunk c in LDS for every wave; stage of c - 1 free
    asm volatile("" ::: "memory");
    if (c + 1 < nch) issue(c + 1, (c + 1) & 1);
    const int st = c & 1;
    f16x8 wa[2], wb[2];
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) {
      const u32x4 raw = *(const u32x4*)(&lw[st][(wv * 2 + ft) * 1024 + 16 * lane]);
      i8x16_to_f16(raw, wa[ft], wb[ft]);
      wa[ft] = wa[ft] * sc[ft];
      wb[ft] = wb[ft] * sc[ft];
    }
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      const f16* xr = &lx[st][(rt * 16 + (lane & 15)) * 64];
      const int p0 = 2 * (lane >> 4);
      const f16x8 fa = *(const f16x8*)(xr + 8 * (p0 ^ sw));
      const f16x8 fb2 = *(const f16x8*)(xr + 8 * ((p0 + 1) ^ sw));
#pragma unroll
      for (int ft = 0; ft < 2; ++ft) {
        acc[ft][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[ft], fa, acc[ft][rt], 0, 0, 0);
        acc[ft][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[ft], fb2, acc[ft][rt], 0, 0, 0);
      }
    }
  }

  // epilogue: lane holds features nb + r (r < 4) of row m for every (ft, rt)
  const bool vec = ((ldy & 3) == 0) && (((uintptr_t)y & 7) == 0) &&
                   (!res || (((ldr & 3) == 0) && (((uintptr_t)res & 7) == 0)));
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    const int m = m0 + rt * 16 + (lane & 15);
    if (m >= M) continue;
    long p_raw = 0;
    if (EPI == GEPI_ROPE) p_raw = ro.pos[m];
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) {
      const int nb = n0 + (wv * 2 + ft) * 16 + 4 * (lane >> 4);
      if (nb >= N) continue;
      f16x4 yv;
#pragma unroll
      for (int r = 0; r < 4; ++r) yv[r] = (f16)acc[ft][rt][r];
      if (EPI == GEPI_STORE) {
        if (vec && nb + 3 < N) {  // one 8-byte store (and residual load) per lane
          if (res) yv = yv + *(const f16x4*)(res + (long)m * ldr + nb);
          *(f16x4*)(y + (long)m * ldy + nb) = yv;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (nb + r < N) {
              f16 o = yv[r];
              if (res) o = o + res[(long)m * ldr + nb + r];
              y[(long)m * ldy + nb + r] = o;
            }
          }
        }
      } else if (EPI == GEPI_ROPE) {  // HD % 4 == 0: the 4 features lie in one head
        const int h = nb / ro.HD, d = nb - h * ro.HD;
        const bool pval = p_raw >= 0 && p_raw < ro.L;
        const long p = p_raw < 0 ? 0 : (p_raw >= ro.L ? ro.L - 1 : p_raw);
        f16x4 o = yv;
        if (h < ro.Hq + ro.Hk) {
          const f32x4 cs = *(const f32x4*)(ro.rope + p * ro.HD + d);
          const float x0 = (float)yv[0], x1 = (float)yv[1], x2 = (float)yv[2], x3 = (float)yv[3];
          o[0] = (f16)(x0 * cs[0] - x1 * cs[1]);
          o[1] = (f16)(x1 * cs[0] + x0 * cs[1]);
          o[2] = (f16)(x2 * cs[2] - x3 * cs[3]);
          o[3] = (f16)(x3 * cs[2] + x2 * cs[3]);
        }
        if (h < ro.Hq) {
          *(f16x4*)(ro.q + ((long)m * ro.Hq + h) * ro.HD + d) = o;
        } else if (pval) {
          const int b = m / ro.S;
          const int kh = h < ro.Hq + ro.Hk ? h - ro.Hq : h - ro.Hq - ro.Hk;
          f16* dst = h < ro.Hq + ro.Hk ? ro.kc : ro.vc;
          *(f16x4*)(dst + (((long)b * ro.Hk + kh) * ro.L + p) * ro.HD + d) = o;
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

template <int EPI, bool RM = false>
static int launch_gemm(const f16* x, long ldx, const int8_t* wp, const f16* s, const f16* res,
                       long ldr, f16* y, long ldy, int M, int N, int K, hipStream_t st,
                       RopeOut ro = RopeOut{}) {
  const int nfb = (N + GT_N - 1) / GT_N;
  const int nmb = (M + GT_M - 1) / GT_M;
  const long blocks = (long)((nfb + 7) / 8) * 8 * nmb;
  if (blocks > 0x7FFFFFFFL) return ECD_ENOTSUP;
  hipLaunchKernelGGL((gemm_i8p_kernel<EPI, RM>), dim3((unsigned)blocks), dim3(256), 0, st, x, ldx,
                     wp, s, res, ldr, y, ldy, M, N, K, nfb, nmb, ro);
  return ecd_launch_status();
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// the per-lane byte offsets of the x loads are 32-bit: the x buffer must stay below 2 GiB
static bool x_offsets_fit(int M, long ldx) { return (long)M * ldx * 2 < 0x7FFFFFFFL; }

// The dense-numerics GEMM on a row-major [N, K] int8 weight (int8_mm with more than 16 rows).
// Returns 1 without launching when the operands do not fit the kernel (the caller then runs
// its own path).
int gemm_i8_rowmajor(const f16* x, long ldx, const int8_t* w, const f16* s, const f16* res,
                     long ldr, f16* y, long ldy, int M, int N, int K, hipStream_t st) {
  if ((K % 64) || (ldx % 8) || !al16(x) || !al16(w) || !x_offsets_fit(M, ldx) ||
      16L * K >= 0x7FFFFFFFL)
    return 1;
  return launch_gemm<GEPI_STORE, true>(x, ldx, w, s, res, ldr, y, ldy, M, N, K, st);
}

}  // namespace ecd

using namespace ecd;

extern "C" {

int ecd_gemm_i8p(const void* x, long ldx, const void* wp, const void* s, const void* res,
                 long ldr, void* y, long ldy, int M, int N, int K, void* stream) {
  if (!x || !wp || !s || !y || M <= 0 || N <= 0 || K <= 0 || (K % 64) || ldx < K || (ldx % 8) ||
      !al16(x) || !al16(wp) || ldy < N || (res && ldr < N))
    return ECD_EINVAL;
  if (!x_offsets_fit(M, ldx)) return ECD_ENOTSUP;
  return launch_gemm<GEPI_STORE>((const f16*)x, ldx, (const int8_t*)wp, (const f16*)s,
                                 (const f16*)res, ldr, (f16*)y, ldy, M, N, K, (hipStream_t)stream);
}

int ecd_gemm_i8p_rope(const void* x, long ldx, const void* wp, const void* s, const float* rope,
                      const int64_t* pos, void* q, void* kc, void* vc, int M, int S, int Hq,
                      int Hk, int L, int HD, int K, void* stream) {
  if (!x || !wp || !s || !rope || !pos || !q || !kc || !vc || M <= 0 || S <= 0 || Hq <= 0 ||
      Hk <= 0 || (Hq % Hk) || L <= 0 || HD <= 0 || (HD % 4) || K <= 0 || (K % 64) || ldx < K ||
      (ldx % 8) || !al16(x) || !al16(wp) || ((uintptr_t)q & 7) || ((uintptr_t)kc & 7) ||
      ((uintptr_t)vc & 7) || ((uintptr_t)rope & 15))
    return ECD_EINVAL;
  if (!x_offsets_fit(M, ldx)) return ECD_ENOTSUP;
  const RopeOut ro{rope, pos, (f16*)q, (f16*)kc, (f16*)vc, S, Hq, Hk, L, HD};
  return launch_gemm<GEPI_ROPE>((const f16*)x, ldx, (const int8_t*)wp, (const f16*)s, nullptr, 0,
                                nullptr, 0, M, (Hq + 2 * Hk) * HD, K, (hipStream_t)stream, ro);
}

int ecd_gemm_i8p_silu(const void* x, long ldx, const void* wp, const void* s, void* mm,
                      long ldm, int M, int F, int K, void* stream) {
  if (!x || !wp || !s || !mm || M <= 0 || F <= 0 || (F % 2) || K <= 0 || (K % 64) || ldx < K ||
      (ldx % 8) || !al16(x) || !al16(wp) || ldm < F || (ldm % 2) || ((uintptr_t)mm & 3))
    return ECD_EINVAL;
  if (!x_offsets_fit(M, ldx)) return ECD_ENOTSUP;
  return launch_gemm<GEPI_SILU>((const f16*)x, ldx, (const int8_t*)wp, (const f16*)s, nullptr,
                                0, (f16*)mm, ldm, M, 2 * F, K, (hipStream_t)stream);
}

}  // extern "C"
