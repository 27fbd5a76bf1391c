// Per-wave flash-decoding core shared by the attention kernels and the attention-prologue GEMV.
// Semantics: app/kernels.py:111-153 (see decode_attn.hip for the full description).
#pragma once
#include "common.h"

namespace ecd {

// One split of one (row, kv head) as seen by one wave: on return lanes 0..15 hold the
// unnormalised accumulators acc[g][j][0..7] of d-chunk 8 (lane + 16 j), and lane g < G holds
// head g's running max m and running sum l (m = -inf, l = 0 for an empty split).
template <int HD, int G>
struct SplitState {
  static constexpr int NDP = (HD + 127) / 128;
  float m_run, l_run;
  float acc[G][NDP][8];
};

// K rows (A operand: lane l holds token t0 + (l & 15), d-chunk 8 (l >> 4) + 32 i) and V rows
// (lane l holds token t0 + 4 (l >> 4) + rr, d-chunk 8 (l & 15) + 128 j) of one 16-token tile.
template <int HD>
struct KVTile {
  static constexpr int NKC = HD / 32;
  static constexpr int NDP = (HD + 127) / 128;
  f16x8 k[NKC];
  f16x8 v[4][NDP];
};

template <bool NT>
__device__ __forceinline__ f16x8 ld_kv8(const f16* p) {
  if (NT) return __builtin_nontemporal_load((const f16x8*)p);
  return *(const f16x8*)p;
}

// Loads the tile at t0 with token indices clamped to `lim` (any valid slot).  Tokens past the
// attended range are masked by attn_run, so a tile may be loaded before that range is known.
// NT: nontemporal loads (the slots are read once per step: they then do not displace what the
// Infinity Cache holds for later launches).
template <int HD, bool NT = false>
__device__ __forceinline__ void kv_load(KVTile<HD>& t, const f16* __restrict__ kb,
                                        const f16* __restrict__ vb, int t0, int lim, int lane) {
  const int row = lane & 15;
  const int grp = lane >> 4;
  const f16* kp = kb + (long)min(t0 + row, lim) * HD + 8 * grp;
#pragma unroll
  for (int i = 0; i < KVTile<HD>::NKC; ++i) t.k[i] = ld_kv8<NT>(kp + 32 * i);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const f16* vp = vb + (long)min(t0 + 4 * grp + rr, lim) * HD + 8 * row;
#pragma unroll
    for (int j = 0; j < KVTile<HD>::NDP; ++j) {
      if (8 * (row + 16 * j) < HD)
        t.v[rr][j] = ld_kv8<NT>(vp + 128 * j);
      else
        t.v[rr][j] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
}

// Online-softmax update of one 16-token tile starting at t0 (tokens >= hi masked).
template <int HD, int G>
__device__ __forceinline__ void attn_tile(SplitState<HD, G>& ss, float& m_run, float& l_run,
                                          const f16x8 (&qf)[HD / 32], KVTile<HD>& cur, int t0,
                                          int hi, float scale, int lane) {
  constexpr int NKC = HD / 32;
  constexpr int NDP = SplitState<HD, G>::NDP;
  const int grp = lane >> 4;
  // V rows past the range contribute nothing (they may hold any bits, even NaN)
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    if (t0 + 4 * grp + rr >= hi)
#pragma unroll
      for (int j = 0; j < NDP; ++j) cur.v[rr][j] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  f32x4 st = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NKC; ++i) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[i], qf[i], st, 0, 0, 0);

  float sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int t = t0 + 4 * grp + rr;
    sc[rr] = (t < hi) ? st[rr] * scale : -INFINITY;
    mx = fmaxf(mx, sc[rr]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_new = fmaxf(m_run, mx);
  const float alpha = __expf(m_run - m_new);
  float pr[4];
  float ps = 0.f;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    pr[rr] = __expf(sc[rr] - m_new);
    ps += pr[rr];
  }
  ps += __shfl_xor(ps, 16, 64);
  ps += __shfl_xor(ps, 32, 64);
  l_run = l_run * alpha + ps;
  m_run = m_new;

#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int src = 16 * grp + g;
    const float ag = __shfl(alpha, src, 64);
    float pg[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) pg[rr] = (float)(f16)__shfl(pr[rr], src, 64);
#pragma unroll
    for (int j = 0; j < NDP; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = ss.acc[g][j][e] * ag;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) a += pg[rr] * (float)cur.v[rr][j][e];
        ss.acc[g][j][e] = a;
      }
  }
}

// The split [lo, hi) with its first tile already loaded (at lo) into ring[0] (PRE: the first
// RING tiles already in ring[0 .. RING - 1]).  RING tiles are in flight: slot r holds tiles r,
// r + RING, ...; a slot is refilled as soon as its tile is consumed, so the split costs about
// one memory round trip per RING tiles.
template <int HD, int G, int RING, bool PRE = false>
__device__ __forceinline__ void attn_run(SplitState<HD, G>& ss, const f16x8 (&qf)[HD / 32],
                                         KVTile<HD> (&ring)[RING], const f16* __restrict__ kb,
                                         const f16* __restrict__ vb, int lo, int hi, float scale,
                                         int lane) {
  constexpr int NDP = SplitState<HD, G>::NDP;
  float m_run = -INFINITY;
  float l_run = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < NDP; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss.acc[g][j][e] = 0.f;

  const int ntiles = hi > lo ? (hi - lo + 15) / 16 : 0;
#pragma unroll
  for (int r = 1; r < RING; ++r)
    if (!PRE && r < ntiles) kv_load<HD>(ring[r], kb, vb, lo + 16 * r, hi - 1, lane);
  for (int base = 0; base < ntiles; base += RING) {
#pragma unroll
    for (int r = 0; r < RING; ++r) {
      const int i = base + r;
      if (i < ntiles) {
        attn_tile<HD, G>(ss, m_run, l_run, qf, ring[r], lo + 16 * i, hi, scale, lane);
        if (i + RING < ntiles) kv_load<HD>(ring[r], kb, vb, lo + 16 * (i + RING), hi - 1, lane);
      }
    }
  }

  // merge the four token phases (lane groups) of every d-chunk
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < NDP; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = ss.acc[g][j][e];
        a += __shfl_xor(a, 16, 64);
        a += __shfl_xor(a, 32, 64);
        ss.acc[g][j][e] = a;
      }
  ss.m_run = m_run;
  ss.l_run = l_run;
}

template <int HD, int G, int RING>
__device__ __forceinline__ void attn_split(SplitState<HD, G>& ss, const f16x8 (&qf)[HD / 32],
                                           const f16* __restrict__ kb, const f16* __restrict__ vb,
                                           int lo, int hi, float scale, int lane) {
  KVTile<HD> ring[RING];
  if (lo < hi) kv_load<HD>(ring[0], kb, vb, lo, hi - 1, lane);
  attn_run<HD, G, RING>(ss, qf, ring, kb, vb, lo, hi, scale, lane);
}

// Writes head g's normalised output o = acc / l as fp16 (lanes 0..15) to dst[g * HD + d].
template <int HD, int G>
__device__ __forceinline__ void attn_store_o(const SplitState<HD, G>& ss, f16* dst, int lane) {
  const int row = lane & 15;
  const int grp = lane >> 4;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lg = __shfl(ss.l_run, g, 64);
    if (grp == 0) {
#pragma unroll
      for (int j = 0; j < SplitState<HD, G>::NDP; ++j) {
        const int d = 8 * (row + 16 * j);
        if (d < HD) {
          f16x8 ov;
#pragma unroll
          for (int e = 0; e < 8; ++e) ov[e] = (f16)(ss.acc[g][j][e] / lg);
          *(f16x8*)(dst + g * HD + d) = ov;
        }
      }
    }
  }
}

// ---- The same split with the P V product on MFMA.  The score MFMA leaves lane l holding
// P[token 4 (l >> 4) + i][head l & 15], i = 0..3 -- the B operand of a 16x16x16 MFMA as it
// stands -- and the V tile gives lane l the rows d = 128 j + 8 (l & 15) + b (b = 0..7) of tokens
// 4 (l >> 4) + i, i.e. the A operand of V^T for the block of rows {128 j + 8 m + b : m < 16}.
// So P V is 8 NDP MFMAs per tile with no lane exchange, and the sum over the tile's tokens
// happens inside them.  acc[j][b] is that block's output: lane l holds rows
// m = 4 (l >> 4) + i of head l & 15, i.e. d = 128 j + 8 (4 (l >> 4) + i) + b.
template <int HD, int G>
struct SplitStateM {
  static constexpr int NDP = (HD + 127) / 128;
  float m_run, l_run;  // head l & 15's running max and sum (equal in the four lane groups)
  f32x4 acc[NDP][8];
};

template <int HD, int G>
__device__ __forceinline__ void attn_tile_m(SplitStateM<HD, G>& ss, float& m_run, float& l_run,
                                            const f16x8 (&qf)[HD / 32], KVTile<HD>& cur, int t0,
                                            int hi, float scale, int lane) {
  constexpr int NKC = HD / 32;
  constexpr int NDP = KVTile<HD>::NDP;
  const int grp = lane >> 4;
  // V rows past the range contribute nothing (they may hold any bits, even NaN)
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    if (t0 + 4 * grp + rr >= hi)
#pragma unroll
      for (int j = 0; j < NDP; ++j) cur.v[rr][j] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  f32x4 st = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NKC; ++i) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[i], qf[i], st, 0, 0, 0);

  float sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int t = t0 + 4 * grp + rr;
    sc[rr] = (t < hi) ? st[rr] * scale : -INFINITY;
    mx = fmaxf(mx, sc[rr]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_new = fmaxf(m_run, mx);
  const float alpha = __expf(m_run - m_new);
  float pr[4];
  float ps = 0.f;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    pr[rr] = __expf(sc[rr] - m_new);
    ps += pr[rr];
  }
  ps += __shfl_xor(ps, 16, 64);
  ps += __shfl_xor(ps, 32, 64);
  l_run = l_run * alpha + ps;
  m_run = m_new;

  const f16x4 pb = (f16x4){(f16)pr[0], (f16)pr[1], (f16)pr[2], (f16)pr[3]};
#pragma unroll
  for (int j = 0; j < NDP; ++j)
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const f16x4 va = (f16x4){cur.v[0][j][b], cur.v[1][j][b], cur.v[2][j][b], cur.v[3][j][b]};
      ss.acc[j][b] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, ss.acc[j][b] * alpha, 0, 0, 0);
    }
}

// A tile staged in LDS in kv_load's register order (16 bytes of lane l at src + 1024 j + 16 l:
// K fragments j < 4, V rows j - 4) back into registers (head_dim 128).
__device__ __forceinline__ void kv_unstage(KVTile<128>& t, const unsigned char* src, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) t.k[i] = *(const f16x8*)(src + 1024 * i + 16 * lane);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) t.v[rr][0] = *(const f16x8*)(src + 1024 * (4 + rr) + 16 * lane);
}

// attn_run with the MFMA P V product (same ring of tiles; PRE: the first RING tiles already in
// ring[0 .. RING - 1], else only ring[0]; NT: the tiles it loads nontemporal; STG with lt set:
// tile 2 was staged in LDS at lt and is read from there into its ring slot instead of loaded).
template <int HD, int G, int RING, bool PRE = false, bool NT = false, bool STG = false>
__device__ __forceinline__ void attn_run_m(SplitStateM<HD, G>& ss, const f16x8 (&qf)[HD / 32],
                                           KVTile<HD> (&ring)[RING], const f16* __restrict__ kb,
                                           const f16* __restrict__ vb, int lo, int hi, float scale,
                                           int lane, const unsigned char* lt = nullptr) {
  static_assert(!STG || (HD == 128 && RING == 2), "staged tile: head_dim 128, two-tile ring");
  constexpr int NDP = SplitStateM<HD, G>::NDP;
  float m_run = -INFINITY;
  float l_run = 0.f;
#pragma unroll
  for (int j = 0; j < NDP; ++j)
#pragma unroll
    for (int b = 0; b < 8; ++b) ss.acc[j][b] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int ntiles = hi > lo ? (hi - lo + 15) / 16 : 0;
#pragma unroll
  for (int r = 1; r < RING; ++r)
    if (!PRE && r < ntiles) kv_load<HD, NT>(ring[r], kb, vb, lo + 16 * r, hi - 1, lane);
  for (int base = 0; base < ntiles; base += RING) {
#pragma unroll
    for (int r = 0; r < RING; ++r) {
      const int i = base + r;
      if (i < ntiles) {
        if constexpr (STG) {
          if (lt && i == 2) kv_unstage(*(KVTile<128>*)&ring[r], lt, lane);
        }
        attn_tile_m<HD, G>(ss, m_run, l_run, qf, ring[r], lo + 16 * i, hi, scale, lane);
        if (i + RING < ntiles && !(STG && lt && i + RING == 2))
          kv_load<HD, NT>(ring[r], kb, vb, lo + 16 * (i + RING), hi - 1, lane);
      }
    }
  }
  ss.m_run = m_run;
  ss.l_run = l_run;
}

// Head g's normalised output o = acc / l as fp16 to dst[g * HD + d] (lanes of heads < G); WT:
// agent-scope stores.
template <int HD, int G, bool WT = false>
__device__ __forceinline__ void attn_store_o_m(const SplitStateM<HD, G>& ss, f16* dst, int lane) {
  const int n = lane & 15, grp = lane >> 4;
  if (n >= G) return;
#pragma unroll
  for (int j = 0; j < SplitStateM<HD, G>::NDP; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 128 * j + 8 * (4 * grp + i);
      if (d0 < HD) {
        f16x8 ov;
#pragma unroll
        for (int b = 0; b < 8; ++b) ov[b] = (f16)(ss.acc[j][b][i] / ss.l_run);
        if constexpr (WT) {
          // written through to memory (agent scope): read by other XCDs in the same launch
          const u32x4 u = __builtin_bit_cast(u32x4, ov);
          uint64_t* q = (uint64_t*)(dst + n * HD + d0);
          __hip_atomic_store(q, (uint64_t)u.x | ((uint64_t)u.y << 32), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(q + 1, (uint64_t)u.z | ((uint64_t)u.w << 32), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        } else {
          *(f16x8*)(dst + n * HD + d0) = ov;
        }
      }
    }
}

// Head g's unnormalised partial [m, l, acc[HD]] to p[g * PW ...] (PW >= HD + 2, even).
template <int HD, int G>
__device__ __forceinline__ void attn_store_partial_m(const SplitStateM<HD, G>& ss, float* p,
                                                     int PW, int lane) {
  const int n = lane & 15, grp = lane >> 4;
  if (n >= G) return;
  float* q = p + n * PW;
  if (grp == 0) {
    q[0] = ss.m_run;
    q[1] = ss.l_run;
  }
#pragma unroll
  for (int j = 0; j < SplitStateM<HD, G>::NDP; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 128 * j + 8 * (4 * grp + i);
      if (d0 < HD)
#pragma unroll
        for (int b = 0; b < 8; b += 2)
          *(float2*)(q + 2 + d0 + b) = make_float2(ss.acc[j][b][i], ss.acc[j][b + 1][i]);
    }
}

// Attended length of row r and the [lo, hi) token range of split sp (app/kernels.py:120-127).
__device__ __forceinline__ void split_range(const int64_t* __restrict__ pos, int r, int L,
                                            int nsplit, int sp, int& lo, int& hi) {
  const long praw = pos[r];
  const int ln = (int)(praw + 1 < 0 ? 0 : (praw + 1 > L ? L : praw + 1));
  const int per = (ln + nsplit - 1) / nsplit;
  const int chunk = ((per + 15) / 16) * 16;
  lo = sp * chunk;
  hi = min(ln, lo + chunk);
}

// Q^T fragments of the G query heads of kv head kh (B operand: lane l holds head l & 15,
// d-chunk 8 (l >> 4) + 32 i; zero for heads >= G).
template <int HD, int G>
__device__ __forceinline__ void load_q(f16x8 (&qf)[HD / 32], const f16* __restrict__ q, int r,
                                       int Hq, int kh, int lane) {
  const int row = lane & 15;
  const int grp = lane >> 4;
  const bool gv = row < G;
  const f16* qp = q + ((long)r * Hq + kh * G + (gv ? row : 0)) * HD + 8 * grp;
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) {
    if (gv)
      qf[i] = *(const f16x8*)(qp + 32 * i);
    else
      qf[i] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  }
}

// Short-cache attention of one (row, kv head) pair on one wave, on the VALU (no tiles): lane l
// owns dims [DPL l, DPL l + DPL) of every head (DPL = HD / 64, two per 32-bit word).  kw / vw
// hold slots 0 .. LT - 1 of K and V (slots from n on are ignored whatever their bits, even
// NaN), qw the G query heads.  Scores q . k are summed in fp32 over each lane's dims, then across
// the wave (DPP scans, no branches, so the G x LT sums interleave), scaled, and the softmax is
// the single-block case of app/kernels.py:111-153: m = max of the attended scores, p =
// exp(s - m), l = sum of the unrounded p, acc = sum of fp16(p) v in fp32, o = fp16(acc / l).
// Head g's o goes to dst + g * HD (dst: head 0 of the pair, plus DPL * lane).
template <int HD, int G, int LT>
__device__ __forceinline__ void short_attn_wave(const uint32_t (&kw)[LT][HD / 128],
                                                const uint32_t (&vw)[LT][HD / 128],
                                                const uint32_t (&qw)[G][HD / 128], int n,
                                                float scale, f16* dst) {
  static_assert(HD % 128 == 0 && HD <= 512, "an even number of dims per lane");
  constexpr int DPL = HD / 64;
  constexpr int NW = DPL / 2;
  float sc[G][LT];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < LT; ++t) {
      float a = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const f16x2 qa = __builtin_bit_cast(f16x2, qw[g][w]);
        const f16x2 ka = __builtin_bit_cast(f16x2, kw[t][w]);
        a += (float)qa.x * (float)ka.x;
        a += (float)qa.y * (float)ka.y;
      }
      sc[g][t] = a;
    }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < LT; ++t) sc[g][t] = wave_sum_dpp(sc[g][t]);
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < LT; ++t) sc[g][t] = t < n ? sc[g][t] * scale : -INFINITY;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < LT; ++t) m = fmaxf(m, sc[g][t]);
    float l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
#pragma unroll
    for (int t = 0; t < LT; ++t) {
      const float p = t < n ? __expf(sc[g][t] - m) : 0.f;
      l += p;
      const float ph = (float)(f16)p;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const f16x2 va = __builtin_bit_cast(f16x2, t < n ? vw[t][w] : 0u);
        acc[2 * w] += ph * (float)va.x;
        acc[2 * w + 1] += ph * (float)va.y;
      }
    }
    uint32_t* op = (uint32_t*)(dst + g * HD);
#pragma unroll
    for (int w = 0; w < NW; ++w)
      op[w] = __builtin_bit_cast(uint32_t, (f16x2){(f16)(acc[2 * w] / l), (f16)(acc[2 * w + 1] / l)});
  }
}

}  // namespace ecd
