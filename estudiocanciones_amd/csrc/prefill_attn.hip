// Causal prompt-pass attention on MFMA (gfx950), head_dim 64 or 128.
//
// Semantics (the prompt pass of app/engine.py:123-153, causal SDPA; per-element numerics of
// the decode kernel, app/kernels.py:111-153): row r = b * S + s attends cache slots
// [0, pos[r]] of kv head kh with its G = Hq / Hk query heads; scores fp32(q . k), softmax of
// the scores times scale with a running max (exp2 with scale * log2(e) folded in),
// probabilities rounded to fp16 before the P.V product (fp32 accumulation), the running sum
// over the unrounded fp32 probabilities.
//
// One workgroup of 4 waves per (64 consecutive rows, kv head, batch item); wave w owns rows
// 16 w .. 16 w + 15 for all G heads, lane l the row 16 w + (l & 15).  Per 64-slot tile the
// workgroup stages K (rows as they are, stride HD + 8) and V^T (swizzled words of slot pairs)
// in LDS from coalesced 16-byte loads issued one tile ahead, then each wave computes:
//   S^T = K . Q^T    v_mfma_f32_16x16x32_f16, K fragments from LDS as the A operand (lane l:
//                    slot t0 + 16 j + (l & 15), d = 32 s + 8 (l >> 4)), Q^T as B (held in
//                    registers); lane l ends with the scores of its row for slots
//                    t0 + 16 j + 4 (l >> 4) + i, i < 4;
//   softmax          per row on its 16 lanes' values, reductions across the 4 lane groups;
//                    the mask only on tiles that reach past a row's position, the rescale of
//                    the running state only when a row's maximum grew;
//   O^T += V^T . P^T v_mfma_f32_16x16x32_f16 with P^T as B straight from the softmax registers:
//                    k-slot 8 g + i of a 32-slot step is slot 4 g + i, slot 8 g + 4 + i is
//                    16 + 4 g + i (g = l >> 4), and V^T as A from LDS in the same slot order.
// O^T keeps each lane's row in its column, so the running rescale is lane-local.  Registers
// hold only Q, O^T and one tile of staging loads, so several workgroups share a CU.
//
// With every position set to the last slot (pos[r] = S - 1, cache length S) the same kernel is
// plain non-causal attention over the sequence: the codec estimator's self-attention
// (app/heartcodec/models/transformer.py:117-125, head_dim 64 and 128, one head per kv head).
#include "common.h"

namespace ecd {

constexpr int PA_QB = 64;            // rows per workgroup (4 waves x 16)
constexpr int PA_KT = 64;            // cache slots per tile

// V^T word (d, slot pair w) lives at d * 32 + (w ^ vt_swz(d)): the swizzle keeps word pairs
// together (8-byte fragment reads), puts the fragment reads of a half-wave (16 d rows x 2 lane
// groups) on distinct banks and keeps the staging writes at most 2-way conflicted
__device__ __forceinline__ int vt_swz(int d) { return 4 * (((d >> 1) ^ (d >> 3)) & 7); }

template <int HD, int G>
__global__ __launch_bounds__(256) void prefill_attn_kernel(
    const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
    const int64_t* __restrict__ pos, f16* __restrict__ o, int S, int Hq, int Hk, int L,
    float scale) {
  static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
  constexpr int KS = HD / 32;     // 32-wide k-steps of q . k
  constexpr int DT = HD / 16;     // 16-row d tiles of O^T
  constexpr int KVS = HD + 8;     // LDS row stride of K in halfs: fragment reads conflict-free
  constexpr int DCH = HD / 8;     // 16-byte chunks per cache row
  constexpr int NK = HD / 32;     // K chunks staged per thread per tile (64 x DCH / 256)
  constexpr int NV = HD / 64;     // V (slot pair, chunk) units staged per thread per tile
  __shared__ __align__(16) f16 ks[PA_KT * KVS];
  __shared__ __align__(16) uint32_t vt[HD * (PA_KT / 2)];
  __shared__ int wmax[4];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int kh = blockIdx.y, b = blockIdx.z;
  const int s = blockIdx.x * PA_QB + 16 * wv + col;   // this lane's row within the batch item
  const bool rowok = s < S;
  const long r = (long)b * S + (rowok ? s : 0);
  // attends [0, p] with p clamped to [-1, L - 1]; -1: nothing (no row, or a negative position)
  const long praw = rowok ? pos[r] : -1;
  const int p = praw < 0 ? -1 : (int)min(praw, (long)L - 1);

  // tiles needed by the workgroup: up to the largest attended slot of its rows
  const int pw = (int)wave_max_u32((uint32_t)(p + 1));
  if (lane == 0) wmax[wv] = pw;
  // slots below this are attended by every row of the wave: tiles there need no mask
  const int wfull = (int)wave_min_u32((uint32_t)(p + 1));

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
  const float c2 = scale * 1.44269504088896341f;  // exp(x * scale) = exp2(x * c2)

  // staging loads of one tile, coalesced 16-byte chunks (consecutive threads, consecutive
  // chunks); K chunk c = tid + 256 i is (slot c / DCH, chunk c % DCH), V unit u = tid + 256 i
  // the chunk u % DCH of the slot pair u / DCH.  Slots past the cache are clamped to its last
  // slot (finite values, masked below).
  f16x8 kr[NK], vr[NV][2];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int c = tid + 256 * i;
      kr[i] = *(const f16x8*)(kb + (long)min(t0 + c / DCH, L - 1) * HD + 8 * (c % DCH));
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = tid + 256 * i;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        vr[i][h] = *(const f16x8*)(vb + (long)min(t0 + 2 * (u / DCH) + h, L - 1) * HD + 8 * (u % DCH));
    }
  };
  // K rows as they are; V transposed into words {V[2w][d], V[2w + 1][d]}
  auto stage_tile = [&]() {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int c = tid + 256 * i;
      *(f16x8*)(&ks[(c / DCH) * KVS + 8 * (c % DCH)]) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = tid + 256 * i, w = u / DCH, d0 = 8 * (u % DCH);
      const u32x4 a = __builtin_bit_cast(u32x4, vr[i][0]);
      const u32x4 c = __builtin_bit_cast(u32x4, vr[i][1]);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = d0 + e;
        vt[d * (PA_KT / 2) + (w ^ vt_swz(d))] =
            __builtin_amdgcn_perm(cw[e >> 1], aw[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
      }
    }
  };

  // one tile of 64 slots from LDS: S^T, online softmax, O^T += V^T . P^T
  auto compute_tile = [&](int t0) {
    // S^T: raw scores q . k of this lane's row; slots past its position masked where the tile
    // reaches beyond the wave's shortest row
    f32x4 sacc[G][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x8 kf[KS];
#pragma unroll
      for (int st = 0; st < KS; ++st)
        kf[st] = *(const f16x8*)(&ks[(16 * j + col) * KVS + 32 * st + 8 * grp]);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < KS; ++st)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[st], qf[g][st], acc, 0, 0, 0);
        sacc[g][j] = acc;
      }
    }
    if (t0 + PA_KT > wfull) {  // wave-uniform: some row of the wave ends inside this tile
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t0 + 16 * j + 4 * grp + i > p) sacc[g][j][i] = -INFINITY;
    }

    // online softmax per (row, head) over the scaled scores: exp(s*scale - m*scale) as
    // exp2(s*c2 - m*c2) with m the running maximum of the raw scores (scale > 0); the running
    // state is rescaled only when a row's maximum grew
    f16x8 pb[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sacc[g][j][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[g], mx);
      const float mb = m_new == -INFINITY ? 0.f : m_new * c2;  // no slot attended yet: p = 0
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[g][j][i], c2, -mb));
          ps += pr;
          pb[g][j >> 1][4 * (j & 1) + i] = (f16)pr;
        }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      if (__any(m_new != m_run[g])) {  // alpha = 1 exactly where the maximum did not move
        asm volatile("" ::: "memory");  // keep this a branch: most tiles skip it
        const float alpha = __builtin_amdgcn_exp2f(m_run[g] * c2 - mb);
        l_run[g] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[g][dt] = oacc[g][dt] * alpha;
      }
      l_run[g] += ps;
      m_run[g] = m_new;
    }

    // O^T += V^T . P^T: A fragment (d = 16 dt + col, slots 32 ks + 4 grp + i, 32 ks + 16 + 4 grp + i)
#pragma unroll
    for (int kq = 0; kq < 2; ++kq)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + col, w = 16 * kq + 2 * grp, sw = vt_swz(d);
        const u32x2 lo = *(const u32x2*)(&vt[d * (PA_KT / 2) + (w ^ sw)]);
        const u32x2 hi = *(const u32x2*)(&vt[d * (PA_KT / 2) + ((w + 8) ^ sw)]);
        const f16x8 va8 = __builtin_bit_cast(f16x8, (u32x4){lo.x, lo.y, hi.x, hi.y});
#pragma unroll
        for (int g = 0; g < G; ++g)
          oacc[g][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va8, pb[g][kq], oacc[g][dt], 0, 0, 0);
      }
  };

  // the next tile's staging loads are in flight while this one is computed
  if (ntiles > 0) load_tile(0);
  for (int it = 0; it < ntiles; ++it) {
    const int t0 = it * PA_KT;
    stage_tile();
    if (it + 1 < ntiles) load_tile(t0 + PA_KT);
    __syncthreads();  // K and V^T of this tile complete
    compute_tile(t0);
    __syncthreads();  // consumed before the next tile overwrites them
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
      ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15) || ((uintptr_t)o & 7) || !(scale > 0.f))
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
