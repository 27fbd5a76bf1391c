// Causal prompt-pass attention on MFMA (gfx950), head_dim 64 or 128.
//
// Semantics (the prompt pass of app/engine.py:123-153, causal SDPA; per-element numerics of
// the decode kernel, app/kernels.py:111-153): row r = b * S + s attends cache slots
// [0, pos[r]] of kv head kh with its G = Hq / Hk query heads; scores fp32(q . k) * scale, a
// running max and natural exp, probabilities rounded to fp16 before the P.V product (fp32
// accumulation), the running sum over the unrounded fp32 probabilities.
//
// One workgroup of 4 waves per (64 consecutive rows, kv head, batch item); wave w owns rows
// 16 w .. 16 w + 15 for all G heads, lane l the row 16 w + (l & 15).  Per 64-slot tile:
//   S^T = K . Q^T    v_mfma_f32_16x16x32_f16, K rows as the A operand straight from the cache
//                    (lane l: slot t0 + 16 j + (l & 15), 16 bytes at d = 32 s + 8 (l >> 4)), Q^T
//                    as B (held in registers); lane l ends with the scores of its row for slots
//                    t0 + 16 j + 4 (l >> 4) + i, i < 4;
//   softmax          per row on its 16 lanes' values, reductions across the 4 lane groups;
//   O^T += V^T . P^T v_mfma_f32_16x16x32_f16 with P^T as B straight from the softmax registers:
//                    k-slot 8 g + i of a 32-slot step is slot 4 g + i, slot 8 g + 4 + i is
//                    16 + 4 g + i (g = l >> 4), and V^T as A read from LDS with the same slot
//                    order (V staged transposed, [d][slot], by the whole workgroup).
// O^T keeps each lane's row in its column, so the running rescale is lane-local.
//
// With every position set to the last slot (pos[r] = S - 1, cache length S) the same kernel is
// plain non-causal attention over the sequence: the codec estimator's self-attention
// (app/heartcodec/models/transformer.py:117-125, head_dim 64 and 128, one head per kv head).
#include "common.h"

namespace ecd {

constexpr int PA_QB = 64;            // rows per workgroup (4 waves x 16)
constexpr int PA_KT = 64;            // cache slots per tile
constexpr int PA_VS = PA_KT + 8;     // LDS row stride of V^T in halfs (spreads the banks)

template <int HD, int G>
__global__ __launch_bounds__(256) void prefill_attn_kernel(
    const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
    const int64_t* __restrict__ pos, f16* __restrict__ o, int S, int Hq, int Hk, int L,
    float scale) {
  static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
  constexpr int KS = HD / 32;   // 32-wide k-steps of q . k
  constexpr int DT = HD / 16;   // 16-row d tiles of O^T
  constexpr int DPT = HD / 8;   // d values per thread in the V staging
  __shared__ __align__(16) f16 vt[HD * PA_VS];
  __shared__ int wmax[4];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int kh = blockIdx.y, b = blockIdx.z;
  const int s = blockIdx.x * PA_QB + 16 * wv + col;   // this lane's row within the batch item
  const bool rowok = s < S;
  const long r = (long)b * S + (rowok ? s : 0);
  const int p = rowok ? min((int)pos[r], L - 1) : -1;  // attends [0, p]; -1: no row

  // tiles needed by the workgroup: up to the largest attended slot of its rows
  const int pw = (int)wave_max_u32((uint32_t)(p + 1));
  if (lane == 0) wmax[wv] = pw;

  // Q^T fragments: head g, k-step st -> row r, d = 32 st + 8 grp .. +7
  f16x8 qf[G][KS];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int st = 0; st < KS; ++st)
      qf[g][st] = *(const f16x8*)(q + r * (long)Hq * HD + (long)(kh * G + g) * HD + 32 * st + 8 * grp);

  f32x4 oacc[G][DT];
  float m_run[G], l_run[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[g][dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();
  const int pmax = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));  // slots attended + 1
  const int ntiles = (pmax + PA_KT - 1) / PA_KT;

  const long cbase = ((long)b * Hk + kh) * (long)L * HD;
  const f16* kb = kc + cbase;
  const f16* vb = vc + cbase;
  // V staging: thread tid transposes slots t0 + 2 (tid >> 3) and +1, d = DPT (tid & 7) .. +DPT-1
  const int vp = 2 * (tid >> 3);
  const int vd = DPT * (tid & 7);

  // loads of one tile: V pair (2 x DPT halfs), this wave's K fragments (4 x KS x 16 B); slots
  // past the cache are clamped to its last slot (finite values, masked below)
  auto load_tile = [&](int t0, f16x8 (&va)[2][DPT / 8], f16x8 (&kf)[4][KS]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f16* src = vb + (long)min(t0 + vp + u, L - 1) * HD + vd;
#pragma unroll
      for (int h = 0; h < DPT / 8; ++h) va[u][h] = *(const f16x8*)(src + 8 * h);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16* src = kb + (long)min(t0 + 16 * j + col, L - 1) * HD + 8 * grp;
#pragma unroll
      for (int st = 0; st < KS; ++st) kf[j][st] = *(const f16x8*)(src + 32 * st);
    }
  };
  // the next tile's loads are issued before this one is computed where registers allow (G <= 3:
  // with 4 heads the second buffer would spill)
  constexpr bool PREFETCH = HD == 64 || G <= 3;
  f16x8 va[2][DPT / 8], kf[4][KS];
  if (PREFETCH && ntiles > 0) load_tile(0, va, kf);

  for (int it = 0; it < ntiles; ++it) {
    const int t0 = it * PA_KT;
    f16x8 vn[2][DPT / 8], kn[4][KS];
    if (!PREFETCH)
      load_tile(t0, va, kf);
    else if (it + 1 < ntiles)
      load_tile(t0 + PA_KT, vn, kn);
    // V^T into LDS: word (d, slot pair) = {V[t][d], V[t + 1][d]}
#pragma unroll
    for (int h = 0; h < DPT / 8; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f16x2 w;
        w.x = va[0][h][e];
        w.y = va[1][h][e];
        *(f16x2*)(&vt[(vd + 8 * h + e) * PA_VS + vp]) = w;
      }

    // S^T and the masked, scaled scores of this lane's row
    float sc[G][4][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < KS; ++st)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[j][st], qf[g][st], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sc[g][j][i] = (t0 + 16 * j + 4 * grp + i <= p) ? acc[i] * scale : -INFINITY;
      }

    // online softmax per (row, head); P^T fragments for the two 32-slot steps
    f16x8 pb[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[g][j][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[g], mx);
      const bool none = m_new == -INFINITY;  // nothing attended yet (rows without a position)
      const float alpha = none ? 1.f : __expf(m_run[g] - m_new);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = none ? 0.f : __expf(sc[g][j][i] - m_new);
          ps += pr;
          pb[g][j >> 1][4 * (j & 1) + i] = (f16)pr;
        }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      l_run[g] = l_run[g] * alpha + ps;
      m_run[g] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[g][dt] = oacc[g][dt] * alpha;
    }
    __syncthreads();  // V^T complete

    // O^T += V^T . P^T: A fragment (d = 16 dt + col, slots 32 ks + 4 grp + i, 32 ks + 16 + 4 grp + i)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f16* vr = &vt[(16 * dt + col) * PA_VS + 32 * ks + 4 * grp];
        f16x8 va8;
        const f16x4 lo = *(const f16x4*)vr;
        const f16x4 hi = *(const f16x4*)(vr + 16);
        va8 = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int g = 0; g < G; ++g)
          oacc[g][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va8, pb[g][ks], oacc[g][dt], 0, 0, 0);
      }
    __syncthreads();  // V^T consumed before the next tile overwrites it
    if (PREFETCH && it + 1 < ntiles) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int h = 0; h < DPT / 8; ++h) va[u][h] = vn[u][h];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int st = 0; st < KS; ++st) kf[j][st] = kn[j][st];
    }
  }

  // O = O^T / l: lane holds row s, d = 16 dt + 4 grp + i
  if (!rowok) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float inv = l_run[g] > 0.f ? 1.f / l_run[g] : 0.f;
    f16* dst = o + r * (long)Hq * HD + (long)(kh * G + g) * HD + 4 * grp;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      f16x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (f16)(oacc[g][dt][i] * inv);
      *(f16x4*)(dst + 16 * dt) = v;
    }
  }
}

}  // namespace ecd

using namespace ecd;

extern "C" int ecd_prefill_attn(const void* q, const void* kc, const void* vc, const int64_t* pos,
                                void* o, int B, int S, int Hq, int Hk, int L, int HD, float scale,
                                void* stream) {
  if (!q || !kc || !vc || !pos || !o || B <= 0 || S <= 0 || Hk <= 0 || Hq <= 0 || L <= 0 ||
      (Hq % Hk) != 0 || Hq / Hk > 4 || (HD != 64 && HD != 128) || ((uintptr_t)q & 15) ||
      ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15) || ((uintptr_t)o & 7))
    return ECD_EINVAL;
  const int G = Hq / Hk;
  const dim3 grid((S + PA_QB - 1) / PA_QB, Hk, B);
  const hipStream_t st = (hipStream_t)stream;
  const f16 *qh = (const f16*)q, *kh = (const f16*)kc, *vh = (const f16*)vc;
  f16* oh = (f16*)o;
#define PA_LAUNCH(HDV, GV)                                                                    \
  hipLaunchKernelGGL((prefill_attn_kernel<HDV, GV>), grid, dim3(256), 0, st, qh, kh, vh, pos, \
                     oh, S, Hq, Hk, L, scale)
  if (HD == 128) {
    switch (G) {
      case 1: PA_LAUNCH(128, 1); break;
      case 2: PA_LAUNCH(128, 2); break;
      case 3: PA_LAUNCH(128, 3); break;
      default: PA_LAUNCH(128, 4); break;
    }
  } else {
    switch (G) {
      case 1: PA_LAUNCH(64, 1); break;
      case 2: PA_LAUNCH(64, 2); break;
      case 3: PA_LAUNCH(64, 3); break;
      default: PA_LAUNCH(64, 4); break;
    }
  }
#undef PA_LAUNCH
  return ecd_launch_status();
}
