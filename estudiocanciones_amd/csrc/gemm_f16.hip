// fp16-weight GEMM on gfx950 MFMA for the dense layers of the codec's flow-matching estimator
// (the nn.Linear layers and the k = 3 Conv1d-as-GEMM of app/heartcodec/models/transformer.py),
// with torch's F.linear numerics: fp32 accumulation, fp32 bias, one fp16 rounding.
//   EPI_STORE: y = fp16(acc + bias); if alpha != 1, y = fp16(y * alpha); then y = fp16(y + res).
//   EPI_SILU:  weight rows interleaved (gate row j at 2j, up row j at 2j + 1),
//              mm[m, j] = fp16(fp16(silu(g)) * u) with g, u the fp16 GEMM outputs (LlamaMLP,
//              transformer.py:178-181).
//   EPI_PRELU: y = fp16(acc + bias), then nn.PReLU with one slope a: y < 0 -> fp16(a * y), then
//              y = fp16(y + res) (the conv -> PReLU (-> + x) steps of the codec's waveform
//              decoder, app/heartcodec/models/sq_codec.py:149-168).
//
// Packed weights: 16-row tiles x 64-wide K chunks of 2 KB, two 1 KB halves h; lane l's 16 bytes
// of half h hold row l & 15, k = 64c + 16 (l >> 4) + 8h .. +7 (ecd_pack_f16), so one 16-byte
// LDS read is an MFMA A fragment.  The activations x are the B operand.
//
// Tiling (template): 4 waves as WN x WM; wave (wn, wm) owns FT 16-feature tiles and RT 16-row
// tiles of v_mfma_f32_16x16x32_f16, so a block covers BN = 16 WN FT features x BM = 16 WM RT
// rows.  K advances in 64-wide chunks that go straight from global memory into an NS-stage LDS
// ring (LDS DMA, no register staging); x rows are stored with their 16-byte pieces XOR-swizzled
// by row (piece p of row r at position p ^ (r & 7)) so the fragment reads spread over banks.
// At the top of step c each wave waits until its own loads of chunk c have landed (vmcnt counts
// the later chunks still allowed in flight), a barrier publishes the chunk and frees the stage
// read in step c - 1, and then the loads of chunk c + NS - 1 go into that stage.
//
// Why the shapes: every block re-reads its weight tile and x tile from L2 once per chunk, so the
// block tile sets the FLOPs per L2 byte (128 x 128: 64 FLOP/B; 256 x 128: 85 FLOP/B), while the
// number of blocks must still fill 256 CUs; the host picks the tile per shape.
//
// Block order is XCD-aware: the row blocks that share a weight tile get block ids equal modulo 8,
// so they run on one XCD and share its L2 (feature blocks in whole groups of 8; the grid has
// exactly one workgroup per output tile, so narrow outputs launch no empty workgroups).
#include "common.h"

namespace ecd {

enum { F16_STORE = 0, F16_SILU = 1, F16_PRELU = 2, F16_ROPE = 3 };

// wait until at most N vector-memory operations of this wave are outstanding and its LDS
// operations are done (lgkmcnt 0)
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// wait for this wave's DMA of one chunk while the `later` chunks issued after it (uniform,
// 0 .. MAXL) stay in flight; PER instructions per chunk; LGKM: also drain LDS operations
template <int PER, int MAXL, bool LGKM>
__device__ __forceinline__ void wait_chunk(int later) {
  if constexpr (MAXL >= 3) {
    if (later >= 3) { if constexpr (LGKM) wait_vm_lgkm0<3 * PER>(); else wait_vm<3 * PER>(); return; }
  }
  if constexpr (MAXL >= 2) {
    if (later >= 2) { if constexpr (LGKM) wait_vm_lgkm0<2 * PER>(); else wait_vm<2 * PER>(); return; }
  }
  if constexpr (MAXL >= 1) {
    if (later >= 1) { if constexpr (LGKM) wait_vm_lgkm0<PER>(); else wait_vm<PER>(); return; }
  }
  if constexpr (LGKM) wait_vm_lgkm0<0>(); else wait_vm0();
}

// A fragments (two k-halves) of the wave's FT weight tiles and B fragments of its RT row tiles
// for one chunk of LDS stage (lw_st, lx_st).
template <int FT, int RT>
__device__ __forceinline__ void f16_frags(const f16* lw_st, const f16* lx_st, int wn, int wm,
                                          int lane, f16x8 (&wa)[FT], f16x8 (&wb)[FT],
                                          f16x8 (&fa)[RT], f16x8 (&fb)[RT]) {
  const int sw = lane & 7, p0 = 2 * (lane >> 4);
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const f16* tp = lw_st + (wn * FT + ft) * 1024;
    wa[ft] = *(const f16x8*)(tp + 8 * lane);
    wb[ft] = *(const f16x8*)(tp + 512 + 8 * lane);
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const f16* xr = lx_st + ((wm * RT + rt) * 16 + (lane & 15)) * 64;
    fa[rt] = *(const f16x8*)(xr + 8 * (p0 ^ sw));
    fb[rt] = *(const f16x8*)(xr + 8 * ((p0 + 1) ^ sw));
  }
}

// acc[ft][rt] += w[ft] x f[rt] over one k-half; consecutive MFMAs write different accumulators
template <int FT, int RT>
__device__ __forceinline__ void f16_mfma_half(f32x4 (&acc)[FT][RT], const f16x8 (&w)[FT],
                                              const f16x8 (&f)[RT]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
      acc[ft][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[ft], f[rt], acc[ft][rt], 0, 0, 0);
}

// Row layouts of a convolution as a GEMM over implicit tap columns (the waveform decoder):
// row m = b * T + t of the GEMM.  With k > 0, x is time-major with xpad zero rows before each
// sequence and row m's K index j * C + c (C = 64 cpt) reads x row b (T + xpad) + xpad + t + off[j]
// (the tap offsets move the chunk's DMA base; the pad rows supply the zeros of the padding).
// With ypad >= 0, y and res rows are b (T + ypad) + ypad + t.  T = 0: plain rows throughout.
struct RowMap {
  int T, xpad, ypad, cpt, k, rep;
  int off[8];
};

// Output of the q | k | v projection with RoPE (F16_ROPE): features [0, D) are q, [D, 2D) k,
// [2D, 3D) v, D = H * HD, rows m = b * T + t.  q and k pairs (2i, 2i + 1) are rotated by
// tab[t, i] = (cos, sin) (fp16); q goes to rows [M, D], k and v to [B, H, T, HD].
struct RopeOut {
  const f16* tab;
  f16 *q, *k, *v;
  int T, H, HD;
};

__device__ __forceinline__ long seq_row(long m, int T, int pad) {
  const long b = m / T;
  return b * (T + pad) + pad + (m - b * T);
}

// 128 x 128 tiles are built for two waves per SIMD (two blocks per CU); the larger ones for one
template <int EPI, int WN, int WM, int FT, int RT, int NS, bool PL>
__global__ __launch_bounds__(256, (FT * RT <= 16 ? 2 : 1)) void gemm_f16w_kernel(
    const f16* __restrict__ x, long ldx, const f16* __restrict__ wp,
    const float* __restrict__ bias, float alpha, const f16* res, long ldr,
    f16* y, long ldy, int M, int N, int K, int nfb, int nmb, RowMap rm,
    RopeOut ro) {
  static_assert(WN * WM == 4, "four waves");
  constexpr int BN = 16 * WN * FT;      // features per block
  constexpr int BM = 16 * WM * RT;      // rows per block
  constexpr int WI = BN / 16 * 2 / 4;   // weight DMA instructions per wave per chunk (1 KB each)
  constexpr int XI = BM / 8 / 4;        // x DMA instructions per wave per chunk (8 rows each)
  constexpr int PER_CHUNK = WI + XI;
  static_assert(NS >= 2 && NS <= 4 && PER_CHUNK * (NS - 1) < 64, "vmcnt range");
  __shared__ __align__(16) f16 lw[NS][BN / 16 * 1024];  // BN / 16 tiles x 2 KB
  __shared__ __align__(16) f16 lx[NS][BM * 64];         // BM rows x 128 B

  // feature blocks in full groups of 8 share XCDs with their row blocks; the remaining
  // nfb % 8 feature blocks (all of them when nfb < 8) are laid out row-major after them
  const int b = blockIdx.x;
  const int full = nfb & ~7;
  int fb, mb;
  if (b < full * nmb) {
    const int grp8 = b / (8 * nmb);
    const int rem = b - grp8 * 8 * nmb;
    mb = rem >> 3;
    fb = grp8 * 8 + (rem & 7);
  } else {
    const int rem = b - full * nmb;
    const int tw = nfb - full;
    mb = rem / tw;
    fb = full + (rem - mb * tw);
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wv % WN, wm = wv / WN;
  const int n0 = fb * BN;
  const int m0 = mb * BM;
  const int nch = K >> 6;
  const int ntiles = (N + 15) >> 4;
  const long tile_bytes = (long)nch * 2048;

  // DMA sources: weight instruction j of this wave is tile t = i >> 1, half h = i & 1 with
  // i = wv + 4 j (tiles past N re-read the last tile; their results are never stored); x
  // instruction j covers rows 8 i .. 8 i + 7, i = wv + 4 j (rows past M re-read row M - 1).
  const char* wsrc[WI];
  int wdst[WI];
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int i = wv + 4 * j;
    const int t = i >> 1, h = i & 1;
    wsrc[j] = (const char*)wp + (long)min(n0 / 16 + t, ntiles - 1) * tile_bytes + 1024 * h;
    wdst[j] = t * 1024 + 512 * h;  // in halfs
  }
  const uint32_t woff = 16u * lane;
  const int xpiece = (lane & 7) ^ (lane >> 3);
  // with a 2x row-repeat (rm.rep == 2) output step t reads source row (t + o) >> 1 for tap o:
  // (t >> 1) + (o >> 1) for even o, ((t + 1) >> 1) + (o >> 1) for odd o -- two lane rows
  uint32_t xoff[XI], xoff1[XI];
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int i = wv + 4 * j;
    long xr = min(m0 + 8 * i + (lane >> 3), M - 1), xr1 = xr;
    if (rm.k && rm.rep == 2) {
      const long b = xr / rm.T, t = xr - b * rm.T;
      const long base = b * (rm.T / 2 + rm.xpad) + rm.xpad;
      xr = base + (t >> 1);
      xr1 = base + ((t + 1) >> 1);
    } else if (rm.k) {
      xr = xr1 = seq_row(xr, rm.T, rm.xpad);
    }
    xoff[j] = (uint32_t)(xr * ldx * 2 + 16 * xpiece);
    xoff1[j] = (uint32_t)(xr1 * ldx * 2 + 16 * xpiece);
  }
  // chunk c's x base: plain K offset 64 c, or tap j = c / cpt shifted by off[j] rows (by
  // off[j] >> 1 with a 2x row-repeat, odd taps reading the second set of lane rows)
  auto issue = [&](int c, int st) {
#pragma unroll
    for (int j = 0; j < WI; ++j) lds_dma16(wsrc[j] + (long)c * 2048, woff, &lw[st][wdst[j]]);
    const f16* xb = x + (long)c * 64;
    bool odd = false;
    if (rm.k) {
      const int tj = c / rm.cpt;
      int o = rm.off[0];
#pragma unroll
      for (int i = 1; i < 8; ++i)
        if (tj == i) o = rm.off[i];
      odd = rm.rep == 2 && (o & 1);
      xb = x + (long)(rm.rep == 2 ? (o >> 1) : o) * ldx + (long)(c - tj * rm.cpt) * 64;
    }
#pragma unroll
    for (int j = 0; j < XI; ++j)
      lds_dma16(xb, odd ? xoff1[j] : xoff[j], &lx[st][8 * (wv + 4 * j) * 64]);
  };

  f32x4 acc[FT][RT];
#pragma unroll
  for (int ft = 0; ft < FT; ++ft)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[ft][rt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  if constexpr (PL) {
    // Software-pipelined: the fragments of chunk c + 1 are read from LDS while the second
    // k-half MFMAs of chunk c run, and the wait + barrier for chunk c + 1 sit behind the first
    // k-half MFMAs, so no MFMA waits for an LDS read at a chunk boundary.  Chunk c + NS goes
    // into the stage of chunk c (its fragments are in registers by then), so NS - 1 chunks of
    // DMA stay in flight behind the one being computed.
    f16x8 wa0[FT], wb0[FT], fa0[RT], fb0[RT], wa1[FT], wb1[FT], fa1[RT], fb1[RT];
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (s < nch) issue(s, s);
    wait_chunk<PER_CHUNK, NS - 1, false>(min(NS - 1, nch - 1));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    f16_frags<FT, RT>(lw[0], lx[0], wn, wm, lane, wa0, wb0, fa0, fb0);
    // one chunk: MFMAs on (wa, wb, fa, fb) = chunk c, next fragments into (na, nb, nfa, nfb)
#define F16_PL_STEP(c, wa, wb, fa, fb, na, nb, nfa, nfb)                                   \
    do {                                                                                  \
      f16_mfma_half<FT, RT>(acc, wa, fa);                                                 \
      if ((c) + 1 < nch) {                                                                \
        /* own DMA of c + 1 landed (later chunks may fly), own reads of c done */         \
        wait_chunk<PER_CHUNK, NS - 2, true>(min(NS - 2, nch - 2 - (c)));                  \
        asm volatile("" ::: "memory");                                                    \
        __builtin_amdgcn_s_barrier();                                                     \
        asm volatile("" ::: "memory");                                                    \
        if ((c) + NS < nch) issue((c) + NS, (c) % NS);                                    \
        const int sn = ((c) + 1) % NS;                                                    \
        f16_frags<FT, RT>(lw[sn], lx[sn], wn, wm, lane, na, nb, nfa, nfb);                \
      }                                                                                   \
      f16_mfma_half<FT, RT>(acc, wb, fb);                                                 \
    } while (0)
    for (int c = 0; c < nch; c += 2) {
      F16_PL_STEP(c, wa0, wb0, fa0, fb0, wa1, wb1, fa1, fb1);
      if (c + 1 < nch) F16_PL_STEP(c + 1, wa1, wb1, fa1, fb1, wa0, wb0, fa0, fb0);
    }
#undef F16_PL_STEP
  } else {
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nch) issue(s, s);
  for (int c = 0; c < nch; ++c) {
    // chunk c landed for this wave: later chunks c + 1 .. c + NS - 2 may still be in flight
    wait_chunk<PER_CHUNK, NS - 2, false>(min(NS - 2, nch - 1 - c));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // chunk c visible to every wave; stage of c - 1 free
    asm volatile("" ::: "memory");
    if (c + NS - 1 < nch) issue(c + NS - 1, (c + NS - 1) % NS);
    const int st = c % NS;
    f16x8 wa[FT], wb[FT], fa[RT], fb[RT];
    f16_frags<FT, RT>(lw[st], lx[st], wn, wm, lane, wa, wb, fa, fb);
    f16_mfma_half<FT, RT>(acc, wa, fa);
    f16_mfma_half<FT, RT>(acc, wb, fb);
  }
  }

  // epilogue: lane holds features nb .. nb + 3 of row m for every (ft, rt).  Where the rows of
  // y (and res) are 8-byte aligned the four values go out as one 8-byte store.
  const bool vec = ((ldy & 3) == 0) && (((uintptr_t)y & 7) == 0) &&
                   (!res || (((ldr & 3) == 0) && (((uintptr_t)res & 7) == 0)));
  // F16_ROPE: the batch item and time step of each of this lane's row tiles
  int rb[RT], rtm[RT];
  if constexpr (EPI == F16_ROPE) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int mm = min(m0 + (wm * RT + rt) * 16 + (lane & 15), M - 1);
      rb[rt] = mm / ro.T;
      rtm[rt] = mm - rb[rt] * ro.T;
    }
  }
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const int nb = n0 + (wn * FT + ft) * 16 + 4 * (lane >> 4);
    if (nb >= N) continue;
    // F16_ROPE: section (q, k, v), head and offset of this lane's 4 features
    int sec = 0, hc = 0, hh = 0, d = 0;
    if constexpr (EPI == F16_ROPE) {
      const int D = ro.H * ro.HD;
      sec = nb >= 2 * D ? 2 : (nb >= D ? 1 : 0);
      hc = nb - sec * D;
      hh = hc / ro.HD;
      d = hc - hh * ro.HD;
    }
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[r] = bias[min(nb + r, N - 1)];
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int mm = m0 + (wm * RT + rt) * 16 + (lane & 15);
      if (mm >= M) continue;
      const long m = rm.ypad >= 0 ? seq_row(mm, rm.T, rm.ypad) : mm;
      f16x4 yv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        yv[r] = (f16)(acc[ft][rt][r] + bv[r]);
        if (EPI == F16_PRELU) {
          if ((float)yv[r] < 0.f) yv[r] = (f16)((float)yv[r] * alpha);  // alpha: the slope
        } else if (alpha != 1.0f) {
          yv[r] = (f16)((float)yv[r] * alpha);
        }
      }
      if (EPI == F16_STORE || EPI == F16_PRELU) {
        if (vec && nb + 3 < N) {
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
      } else if (EPI == F16_ROPE) {  // 4 features never straddle a head (HD % 4 == 0)
        const int t = rtm[rt];
        if (sec < 2) {
          const f16x4 cs = *(const f16x4*)(ro.tab + (long)t * ro.HD + d);  // pairs d/2, d/2 + 1
          f16 o0, o1, o2, o3;
          rope_pair_f16((float)yv[0], (float)yv[1], (float)cs[0], (float)cs[1], o0, o1);
          rope_pair_f16((float)yv[2], (float)yv[3], (float)cs[2], (float)cs[3], o2, o3);
          yv = (f16x4){o0, o1, o2, o3};
        }
        f16* dst = sec == 0 ? ro.q + m * (ro.H * ro.HD) + hc
                            : (sec == 1 ? ro.k : ro.v) +
                                  (((long)rb[rt] * ro.H + hh) * ro.T + t) * ro.HD + d;
        *(f16x4*)dst = yv;
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

// Pack fp16 w [N, K] into lane-ordered 16 x 64 tiles of 2 KB (two 1 KB halves); with
// `interleave` (N even) packed row 2j is source row j and 2j + 1 is source row N/2 + j.
__global__ __launch_bounds__(256) void pack_f16_kernel(const f16* __restrict__ w, int N, int K,
                                                       int interleave, f16* __restrict__ out) {
  const int nch = K >> 6;
  const long ntiles = (N + 15) >> 4;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= ntiles * nch * 128) return;
  const int l = (int)(idx & 63);
  const int h = (int)((idx >> 6) & 1);
  const long tc = idx >> 7;
  const int c = (int)(tc % nch);
  const long tile = tc / nch;
  const long r = tile * 16 + (l & 15);
  u32x4 v = (u32x4){0u, 0u, 0u, 0u};
  if (r < N) {
    const long src = interleave ? ((r & 1) ? (N >> 1) + (r >> 1) : (r >> 1)) : r;
    v = *(const u32x4*)(w + src * K + 64L * c + 16 * (l >> 4) + 8 * h);
  }
  *(u32x4*)(out + (tile * nch + c) * 1024 + 512 * h + 8 * l) = v;
}

// Tile configurations: {WN, WM, FT, RT, NS}.
//   1: 128 x 128, waves 4 x 1 (32 features x 128 rows each), 2 stages, 64 KB LDS
//   2: 128 x 128, waves 2 x 2 (64 x 64 each), 2 stages, 64 KB
//   3: 256 x 128, waves 4 x 1 (64 x 128 each), 2 stages, 96 KB
//   4: 256 x 128, waves 4 x 1, 3 stages, 144 KB
//   5: 256 x 128, waves 2 x 2 (128 x 64 each), 2 stages, 96 KB
//   6: 128 x 256, waves 2 x 2 (64 x 128 each), 2 stages, 96 KB
//   7: 128 x 128, waves 2 x 2, 3 stages, 96 KB
//   8: as 2, software-pipelined (next chunk's fragments read during this chunk's MFMAs)
//   9: as 1, software-pipelined
//  10: 128 x 64, waves 4 x 1 (32 x 64 each), software-pipelined, 48 KB
//  11: 128 x 64, waves 2 x 2 (64 x 32 each), software-pipelined, 48 KB
//  12: 64 x 128, waves 1 x 4 (64 x 32 each), software-pipelined, 48 KB (outputs <= 64 wide)
//  13: 64 x 256, waves 1 x 4 (64 x 64 each), software-pipelined, 80 KB
//  14: 64 x 64, waves 2 x 2 (32 x 32 each), software-pipelined, 32 KB
//  15: as 14 with 3 stages, 48 KB
//  16: 128 x 96, waves 2 x 2 (64 x 48 each), software-pipelined, 56 KB
template <int EPI, int WN, int WM, int FT, int RT, int NS, bool PL = false>
static int launch_cfg(const f16* x, long ldx, const f16* wp, const float* bias, float alpha,
                      const f16* res, long ldr, f16* y, long ldy, int M, int N, int K,
                      const RowMap& rm, const RopeOut& ro, hipStream_t st) {
  constexpr int BN = 16 * WN * FT, BM = 16 * WM * RT;
  const int nfb = (N + BN - 1) / BN;
  const int nmb = (M + BM - 1) / BM;
  const long blocks = (long)nfb * nmb;
  if (blocks > 0x7FFFFFFFL) return ECD_ENOTSUP;
  hipLaunchKernelGGL((gemm_f16w_kernel<EPI, WN, WM, FT, RT, NS, PL>), dim3((unsigned)blocks),
                     dim3(256), 0, st, x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, nfb,
                     nmb, rm, ro);
  return ecd_launch_status();
}

// Library default per shape (N counts output features before the SiLU pairing).
static int default_cfg(int M, int N, int K, bool silu) {
  // blocks of 128 x 128: below 256 (one per CU) or 512 (the two that fit per CU) a smaller block
  // fills the resident slots that 128 x 128 leaves empty
  const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
  if (silu) return 8;
  if (N <= 64) return 12;                            // the decoder's 64-channel convs
  if (N <= 256 && K >= 4096 && t128 < 256) return 15;  // few blocks, long K: 3 stages in flight
  if (N <= 1536 && t128 < 256) return 14;            // 64 x 64
  if (N <= 1536 && t128 < 512) return 10;            // 128 x 64
  if (N <= 3072 && t128 < 512) return 16;            // 128 x 96
  if (N <= 1024) return 1;                           // the decoder's wider convs over many rows
  return 8;
}

template <int EPI>
static int launch_f16(int cfg, const f16* x, long ldx, const f16* wp, const float* bias,
                      float alpha, const f16* res, long ldr, f16* y, long ldy, int M, int N,
                      int K, const RowMap& rm, const RopeOut& ro, hipStream_t st) {
  if (cfg == 0) cfg = default_cfg(M, N, K, EPI == F16_SILU);
  switch (cfg) {
    case 1: return launch_cfg<EPI, 4, 1, 2, 8, 2>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 2: return launch_cfg<EPI, 2, 2, 4, 4, 2>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 3: return launch_cfg<EPI, 4, 1, 4, 8, 2>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 4: return launch_cfg<EPI, 4, 1, 4, 8, 3>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 5: return launch_cfg<EPI, 2, 2, 8, 4, 2>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 6: return launch_cfg<EPI, 2, 2, 4, 8, 2>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 7: return launch_cfg<EPI, 2, 2, 4, 4, 3>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 8: return launch_cfg<EPI, 2, 2, 4, 4, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 9: return launch_cfg<EPI, 4, 1, 2, 8, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 10: return launch_cfg<EPI, 4, 1, 2, 4, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 11: return launch_cfg<EPI, 2, 2, 4, 2, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 12: return launch_cfg<EPI, 1, 4, 4, 2, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 13: return launch_cfg<EPI, 1, 4, 4, 4, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 14: return launch_cfg<EPI, 2, 2, 2, 2, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 15: return launch_cfg<EPI, 2, 2, 2, 2, 3, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    case 16: return launch_cfg<EPI, 2, 2, 4, 3, 2, true>(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro, st);
    default: return ECD_EINVAL;
  }
}

static int launch_epi(int epi, int cfg, const f16* x, long ldx, const f16* wp, const float* bias,
                      float alpha, const f16* res, long ldr, f16* y, long ldy, int M, int N, int K,
                      const RowMap& rm, hipStream_t st) {
  const RopeOut ro = {nullptr, nullptr, nullptr, nullptr, 1, 1, 4};
  if (epi == F16_SILU)
    return launch_f16<F16_SILU>(cfg, x, ldx, wp, nullptr, 1.0f, nullptr, 0, y, ldy, M, N, K, rm,
                                ro, st);
  if (epi == F16_PRELU)
    return launch_f16<F16_PRELU>(cfg, x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro,
                                 st);
  return launch_f16<F16_STORE>(cfg, x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, rm, ro,
                               st);
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// the per-lane byte offsets of the x loads are 32-bit: the x buffer must stay below 2 GiB
static bool x_offsets_fit(int M, long ldx) { return (long)M * ldx * 2 < 0x7FFFFFFFL; }

}  // namespace ecd

using namespace ecd;

extern "C" {

long ecd_packed_bytes_f16(int N, int K) { return (long)((N + 15) / 16) * 16 * (long)K * 2; }

int ecd_pack_f16(const void* w, int N, int K, int interleave, void* out, void* stream) {
  if (!w || !out || N <= 0 || K <= 0 || (K % 64) || (interleave && (N & 1)) || !al16(w) ||
      !al16(out))
    return ECD_EINVAL;
  const long total = (long)((N + 15) / 16) * (K / 64) * 128;
  hipLaunchKernelGGL(pack_f16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)w, N, K, interleave, (f16*)out);
  return ecd_launch_status();
}

int ecd_gemm_f16p_tuned(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                        const void* res, long ldr, void* y, long ldy, int M, int N, int K,
                        int epi, int cfg, void* stream) {
  if (!x || !wp || !y || M <= 0 || N <= 0 || K <= 0 || (K % 64) || ldx < K || (ldx % 8) ||
      !al16(x) || !al16(wp) || cfg < 0 || cfg > 16 || epi < 0 || epi > 2)
    return ECD_EINVAL;
  const bool silu = epi == F16_SILU;
  if (silu) {
    if ((N % 2) || ldy < N / 2 || (ldy % 2) || ((uintptr_t)y & 3) || bias || res || alpha != 1.0f)
      return ECD_EINVAL;
  } else if (ldy < N || (res && ldr < N)) {
    return ECD_EINVAL;
  }
  if (!x_offsets_fit(M, ldx)) return ECD_ENOTSUP;
  const RowMap rm = {0, 0, -1, 0, 0, 1, {0, 0, 0, 0, 0, 0, 0, 0}};
  return launch_epi(epi, cfg, (const f16*)x, ldx, (const f16*)wp, bias, alpha, (const f16*)res,
                    ldr, (f16*)y, ldy, M, N, K, rm, (hipStream_t)stream);
}

int ecd_gemm_f16p_rope(const void* x, long ldx, const void* wp, const float* bias,
                       const void* tab, void* q, void* k, void* v, int M, int T, int H, int HD,
                       int K, void* stream) {
  const long N = 3L * H * HD;
  if (!x || !wp || !tab || !q || !k || !v || M <= 0 || T <= 0 || M % T || H <= 0 || HD <= 0 ||
      (HD % 4) || N > 0x7FFFFFFFL || K <= 0 || (K % 64) || ldx < K || (ldx % 8) || !al16(x) ||
      !al16(wp) || ((uintptr_t)tab & 7) || ((uintptr_t)q & 7) || ((uintptr_t)k & 7) ||
      ((uintptr_t)v & 7))
    return ECD_EINVAL;
  if (!x_offsets_fit(M, ldx)) return ECD_ENOTSUP;
  const RowMap rm = {0, 0, -1, 0, 0, 1, {0, 0, 0, 0, 0, 0, 0, 0}};
  const RopeOut ro = {(const f16*)tab, (f16*)q, (f16*)k, (f16*)v, T, H, HD};
  return launch_f16<F16_ROPE>(0, (const f16*)x, ldx, (const f16*)wp, bias, 1.0f, nullptr, 0,
                              nullptr, 0, M, (int)N, K, rm, ro, (hipStream_t)stream);
}

int ecd_gemm_f16p_conv_tuned(const void* x, long ldx, const void* wp, const float* bias,
                             float alpha, const void* res, long ldr, void* y, long ldy, int M,
                             int N, int K, int T, int xpad, int ypad, const int* offsets, int k,
                             int rep, int epi, int cfg, void* stream) {
  if (!x || !wp || !y || M <= 0 || N <= 0 || K <= 0 || (K % 64) || (ldx % 8) || !al16(x) ||
      !al16(wp) || epi < 0 || epi > 2 || epi == F16_SILU || cfg < 0 || cfg > 16 || T <= 0 ||
      M % T || k < 0 || k > 8 ||
      (k && (!offsets || K % (64 * k) || xpad < 0)) || (!k && ldx < K) || ldy < N ||
      (res && ldr < N) || ypad < -1 || (rep != 1 && rep != 2) || (rep == 2 && (!k || T % 2)))
    return ECD_EINVAL;
  RowMap rm = {T, xpad, ypad, k ? K / (64 * k) : 0, k, rep, {0, 0, 0, 0, 0, 0, 0, 0}};
  if (k) {
    if (ldx < K / k) return ECD_EINVAL;
    for (int j = 0; j < k; ++j) {
      // source rows stay in the pad rows: shift o (or o >> 1 and (o + 1) >> 1 with a repeat)
      const int lo = rep == 2 ? offsets[j] >> 1 : offsets[j];
      const int hi = rep == 2 ? (offsets[j] + 1) >> 1 : offsets[j];
      if (lo < -xpad || hi > xpad) return ECD_EINVAL;
      rm.off[j] = offsets[j];
    }
  }
  const long tin = rep == 2 ? T / 2 : T;  // source rows per sequence
  const long xrows = k ? (long)(M / T) * (tin + xpad) + xpad : M;  // + the rows after the last
  if (!x_offsets_fit((int)min(xrows, 0x7FFFFFFFL), ldx)) return ECD_ENOTSUP;
  return launch_epi(epi, cfg, (const f16*)x, ldx, (const f16*)wp, bias, alpha, (const f16*)res,
                    ldr, (f16*)y, ldy, M, N, K, rm, (hipStream_t)stream);
}

int ecd_gemm_f16p_conv(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                       const void* res, long ldr, void* y, long ldy, int M, int N, int K, int T,
                       int xpad, int ypad, const int* offsets, int k, int rep, int epi,
                       void* stream) {
  return ecd_gemm_f16p_conv_tuned(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, T, xpad,
                                  ypad, offsets, k, rep, epi, 0, stream);
}

int ecd_gemm_f16p(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                  const void* res, long ldr, void* y, long ldy, int M, int N, int K,
                  void* stream) {
  return ecd_gemm_f16p_tuned(x, ldx, wp, bias, alpha, res, ldr, y, ldy, M, N, K, 0, 0, stream);
}

int ecd_gemm_f16p_prelu(const void* x, long ldx, const void* wp, const float* bias, float slope,
                        const void* res, long ldr, void* y, long ldy, int M, int N, int K,
                        void* stream) {
  return ecd_gemm_f16p_tuned(x, ldx, wp, bias, slope, res, ldr, y, ldy, M, N, K, F16_PRELU, 0,
                             stream);
}

int ecd_gemm_f16p_silu(const void* x, long ldx, const void* wp, void* mm, long ldm, int M, int F,
                       int K, void* stream) {
  if (F <= 0) return ECD_EINVAL;
  return ecd_gemm_f16p_tuned(x, ldx, wp, nullptr, 1.0f, nullptr, 0, mm, ldm, M, 2 * F, K, 1, 0,
                             stream);
}

}  // extern "C"
