// Fused CFG + top-k + temperature sampler over the 8197 codebook logits (gfx950).
//
// Reference (app/engine.py:291-305), per take n of N (rows n = cond, n + N = uncond):
//   l   = fp16( u + fp16( fp16(c - u) * cfg ) )         if CFG (B == 2N), else the logits
//   x   = fp32(l) / temp
//   thr = k-th largest x;  x = x < thr ? -inf : x        (ties with thr are kept)
//   p   = softmax(log_softmax(x))                        (both in fp32)
//   tok = argmax(p / q),  q ~ Exponential(1)             (first index on ties)
//   the token is written for row n and, with CFG, for row n + N.
//
// One block of 1024 threads per take; the selection works on order-preserving 16-bit keys of the
// fp16 logits: x = fp32(l)/temp is strictly monotonic in l, so the threshold and its ties are
// those of l.  Only the kept values (key >= threshold, k of them plus ties) reach the softmax
// and the race: every other index has p = 0 exactly and can neither win nor change a sum.
//   - The k-th largest key: the block's largest key fixes a window of the 16 top-byte digits
//     below it (about 4 octaves); one LDS bin per key of the window (4096) counts the keys that
//     fall there (fine bins: the atomics rarely collide), and a block-wide scan of the bin
//     counts from the top (4 bins per thread) finds where the count reaches k.  When fewer
//     than k keys lie in the window, a two-pass radix select over all keys (8-bit digits)
//     finds the threshold instead.
//   - The kept values land in LDS in descending key order (first slot of each key from the
//     walk, then one atomic per value).  Values with equal keys are equal, so the fp32 sums
//     below see the same sequence of numbers whatever the order among them: results are
//     deterministic.  One wave finishes the softmax and the race without further barriers.
// The Exponential(1) draws are q = -log(u), u = (bits >> 8 + 0.5) * 2^-24 from the
// counter-based Philox4x32-10 generator (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011), keyed by a 64-bit seed read from device memory and
// countered by (vocab index / 4, take, frame position, salt): graph replays at different
// frame positions draw fresh numbers without any mutable RNG state.  Tests can inject the
// draws instead (noise [N, V] fp32).
#include "attn_core.h"

namespace ecd {

__device__ __forceinline__ uint32_t mulhilo(uint32_t a, uint32_t b, uint32_t& hi) {
  const uint64_t p = (uint64_t)a * (uint64_t)b;
  hi = (uint32_t)(p >> 32);
  return (uint32_t)p;
}

// Philox4x32 with 10 rounds (published constants of the Random123 family).
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    uint32_t hi0, hi1;
    const uint32_t lo0 = mulhilo(0xD2511F53u, c[0], hi0);
    const uint32_t lo1 = mulhilo(0xCD9E8D57u, c[2], hi1);
    const uint32_t n0 = hi1 ^ c[1] ^ k0;
    const uint32_t n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

constexpr int SMP_THREADS = 1024;
constexpr int SMP_MAXV = 8704;  // values per take supported (8197 codebook entries + slack)
constexpr int SMP_PER = 9;      // values per thread: 8 contiguous + one of the tail past 8192
constexpr int SMP_WDIG = 16;    // top key bytes (digits) covered by the window below the maximum
constexpr int SMP_WBINS = SMP_WDIG * 256;  // one bin per 16-bit key of the window
// LDS position of window bin b: 4 words of padding after every 64 bins, so that the 64 lanes
// reading their own 64-bin runs as 16-byte words spread over the banks
constexpr int SMP_WBINS_LDS = SMP_WBINS + 4 * (SMP_WBINS / 64);
__device__ __forceinline__ int wbin_at(uint32_t b) { return (int)(b + 4 * (b >> 6)); }

// Order-preserving 16-bit key of an fp16 value (-0.0 must be canonicalised to +0.0 first so
// that key order equals float comparison), and its inverse.
__device__ __forceinline__ uint32_t hkey(f16 h) {
  const uint32_t u = __builtin_bit_cast(uint16_t, h);
  return (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
}
__device__ __forceinline__ f16 hkey_inv(uint32_t k) {
  const uint16_t u = (uint16_t)((k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu));
  return __builtin_bit_cast(f16, u);
}

// vocabulary index of slot j of thread tid
__device__ __forceinline__ int slot_index(int tid, int j) {
  return j < 8 ? 8 * tid + j : 8 * SMP_THREADS + tid;
}

// Digit d (from the top) of the radix select: the largest digit whose cumulative count from
// the top reaches `rank`.  Run by wave 0 over 256 bins; writes (prefix | d << shift, new rank).
__device__ __forceinline__ void radix_pick(const uint32_t* hist, uint32_t* sel, uint32_t prefix,
                                           int shift, int lane) {
  const uint32_t rank = sel[1];
  uint32_t c4 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) c4 += hist[255 - (lane * 4 + j)];
  uint32_t incl = c4;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  const uint32_t excl = incl - c4;
  if (excl < rank && incl >= rank) {
    uint32_t acc = excl;
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = 255 - (lane * 4 + j);
      const uint32_t h = hist[d];
      if (acc + h >= rank) {
        sel[0] = prefix | (d << shift);
        sel[1] = rank - acc;
        break;
      }
      acc += h;
    }
  }
}

// Fallback when fewer than k values lie in the window: the k-th largest key by a two-pass radix
// select over all keys (8-bit digits, LDS histograms), then the kept keys (>= threshold) are
// compacted in (thread, slot) order by prefix sums.  Returns the kept count.
__device__ uint32_t select_full(const uint32_t (&key)[SMP_PER], const f16 (&lv)[SMP_PER],
                                float temp, int topk, uint32_t (&hist)[2][256], uint32_t* sel,
                                uint32_t* wtot, int* kept_i, float* kept_x) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid < 256) {
    hist[0][tid] = 0u;
    hist[1][tid] = 0u;
  }
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = (uint32_t)topk;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j)
    if (key[j]) atomicAdd(&hist[0][key[j] >> 8], 1u);
  __syncthreads();
  if (tid < 64) radix_pick(hist[0], sel, 0u, 8, lane);
  __syncthreads();
  const uint32_t hi8 = sel[0];
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j)
    if (key[j] && (key[j] & 0xFF00u) == hi8) atomicAdd(&hist[1][key[j] & 255u], 1u);
  __syncthreads();
  if (tid < 64) radix_pick(hist[1], sel, hi8, 0, lane);
  __syncthreads();
  const uint32_t thr = sel[0];

  int cnt = 0;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) cnt += (key[j] && key[j] >= thr) ? 1 : 0;
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) wtot[wv] = (uint32_t)incl;
  __syncthreads();
  int base = incl - cnt;
  int total = 0;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) {
    const int t = (int)wtot[w];
    base += w < wv ? t : 0;
    total += t;
  }
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    if (key[j] && key[j] >= thr) {
      kept_i[base] = slot_index(tid, j);
      kept_x[base] = (float)lv[j] / temp;
      ++base;
    }
  }
  return (uint32_t)total;
}

// What the sampler of a depth-decoder pass also does for the next pass, with the sampled token
// t of take n (rows n and n + N with CFG):
//  * rows != NULL: x rows <- rows[t] (the next pass's input, precomputed per token);
//  * qkv != NULL: that pass's layer 0 up to its attention output: q | k | v of the token at
//    slot p (precomputed per token, RoPE applied) -> the cache slot p of kc / vc, and the
//    decode attention over slots 0 .. p (app/kernels.py:110-153: fp32 scores, exp, fp16 P,
//    fp32 P V, o = acc / l) -> o rows.  One wave per (row, kv head) pair, its cached slots
//    0 .. p - 1 loaded while the sampler runs: head_dim 128 into LDS (LDS DMA, at kernel start),
//    head_dim 384 into the wave's registers (86 KB for 8 pairs would not fit beside the
//    sampler's LDS), with the arithmetic of the standalone short-cache kernel.
constexpr int NXA_HD = 128;   // head_dim of the LDS form
constexpr int NXA_SLOTS = 16; // cache slots it reads at most (p < 16)
constexpr int NXA_PAIRS = 4;  // (row, kv head) pairs per take at most
constexpr int NXA_G = 4;      // query heads per kv head at most
constexpr int NXV_HD = 384;   // head_dim of the register form
constexpr int NXV_SLOTS = 8;  // cache slots it holds (p < 8)
constexpr int NXV_PAIRS = 8;  // pairs per take at most (waves 1 .. 8)
constexpr int NXV_G = 2;      // query heads per kv head (the reference decoder's 8 / 4)
struct NextPass {
  const f16* rows;
  long rows_ld;
  f16* x;
  long x_ld;
  int D;
  const f16* qkv;  // [>= V, (Hq + 2 Hk) * HD]: q heads | k heads | v heads per token
  long qkv_ld;
  f16* kc;         // [B, Hk, L, HD]
  f16* vc;
  int L, p;
  f16* o;          // [B, Hq * HD]
  long o_ld;
  int Hq, Hk, HD;
  float scale;
  const f16* ev;   // rows copied as they are, independent of the token: ev row r -> xe row r
  long ev_ld;      // (D wide; the depth decoder's first pass: the projected backbone state)
  f16* xe;
  long xe_ld;
};

// Pair (row, kv head) of the next pass's layer-0 attention for the sampled token tok, one wave:
// q | k | v of the token from its precomputed row (zeros if no index won), k and v into cache
// slot p and LDS slot p (slots 0 .. p - 1 are in LDS already), then scores (lane: head
// lane / 16, slot lane % 16), softmax over the slots of each head, P V (lane: head lane / 16,
// columns 8 (lane % 16) .. + 7) and o.
__device__ __forceinline__ void next_attention(const NextPass& nx, int tok, int V, int aj,
                                               int row, int kh, long cache, int lane,
                                               f16 (*ak)[NXA_HD], f16 (*av)[NXA_HD],
                                               f16 (*aq)[NXA_HD], float (*ape)[NXA_SLOTS]) {
  const int G = nx.Hq / nx.Hk, p = nx.p;
  const bool valid = (uint32_t)tok < (uint32_t)V;
  const f16* src = nx.qkv + (long)(valid ? tok : 0) * nx.qkv_ld;
  // chunk c (16 bytes) of lane: c = lane + 64 u; q heads first, then k, then v of head kh.
  // All loads go out first; one wait covers them and the LDS DMA of the cached slots issued at
  // kernel start, and the stores after it are not waited for.
  const int nq = G * (NXA_HD / 8);  // 16-byte chunks of the pair's q heads
  const int nc = nq + NXA_HD / 4;   // plus k and v
  static_assert(NXA_G * (NXA_HD / 8) + NXA_HD / 4 <= 128, "two chunks per lane");
  f16x8 v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = lane + 64 * u;
    const bool isq = c < nq, isk = !isq && c < nq + NXA_HD / 8;
    const int d = isq ? 0 : 8 * (c - nq - (isk ? 0 : NXA_HD / 8));
    const long so = isq ? (long)kh * G * NXA_HD + 8 * c
                        : (long)(nx.Hq + (isk ? 0 : nx.Hk) + kh) * NXA_HD + d;
    v[u] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    if (valid && c < nc) v[u] = *(const f16x8*)(src + so);
  }
  wait_vm0();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = lane + 64 * u;
    if (c >= nc) continue;
    const bool isq = c < nq, isk = !isq && c < nq + NXA_HD / 8;
    const int d = isq ? 0 : 8 * (c - nq - (isk ? 0 : NXA_HD / 8));
    if (isq) {
      *(f16x8*)(&aq[0][0] + 8 * c) = v[u];
    } else {
      *(f16x8*)(&(isk ? ak : av)[p][d]) = v[u];
      *(f16x8*)((isk ? nx.kc : nx.vc) + cache + (long)p * NXA_HD + d) = v[u];
    }
  }
  const int g = lane >> 4, t = lane & 15;
  const bool on = g < G && t <= p;
  float s = -INFINITY;
  if (on) {
    float acc = 0.f;
#pragma unroll 4
    for (int c = 0; c < NXA_HD / 8; ++c) {
      const f16x8 qv = *(const f16x8*)(&aq[g][8 * c]);
      const f16x8 kv = *(const f16x8*)(&ak[t][8 * c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)qv[e] * (float)kv[e];
    }
    s = acc * nx.scale;
  }
  float m = s;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float pe = on ? expf(s - m) : 0.f;
  float l = pe;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o, 64);
  if (g < G) ape[g][t] = (float)(f16)pe;  // P in fp16 for the P V product
  if (g < G) {
    const int d0 = 8 * (lane & 15);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int u = 0; u <= p; ++u) {
      const float w = ape[g][u];
      const f16x8 vv = *(const f16x8*)(&av[u][d0]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += w * (float)vv[e];
    }
    f16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = (f16)(acc[e] / l);
    *(f16x8*)(nx.o + (long)row * nx.o_ld + (long)(kh * G + g) * NXA_HD + d0) = ov;
  }
  (void)aj;
}

// A D-wide fp16 row (D <= 512 SMP_RCH, a multiple of 8) copied by one wave: every load issued
// before the first store (one memory round trip), 16 bytes per lane and chunk; zeros when
// `valid` is false.
constexpr int SMP_RCH = 6;  // 16-byte chunks per lane: rows up to 3072 wide
__device__ __forceinline__ void row_load(f16x8 (&v)[SMP_RCH], const f16* src, int D, bool valid,
                                         int lane) {
#pragma unroll
  for (int i = 0; i < SMP_RCH; ++i) {
    const int c = 8 * lane + 512 * i;
    v[i] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    if (valid && c < D) v[i] = *(const f16x8*)(src + c);
  }
}
__device__ __forceinline__ void row_store(const f16x8 (&v)[SMP_RCH], f16* d0, f16* d1, int D,
                                          int lane) {
#pragma unroll
  for (int i = 0; i < SMP_RCH; ++i) {
    const int c = 8 * lane + 512 * i;
    if (c < D) {
      *(f16x8*)(d0 + c) = v[i];
      if (d1) *(f16x8*)(d1 + c) = v[i];
    }
  }
}

// The register form's cached slots: lane l holds dims [HD / 64 l, HD / 64 (l + 1)) of slots
// 0 .. NXV_SLOTS - 1 of K and V (the slots from p on are filled or masked later).
template <int HD>
struct NxvSlots {
  uint32_t k[NXV_SLOTS][HD / 128], v[NXV_SLOTS][HD / 128];
};

// A lane's HD / 64 halves (NW 32-bit words) of one row as one load (dwordx3 for head_dim 384):
// one memory instruction per row instead of NW.
template <int NW>
__device__ __forceinline__ void ld_words(uint32_t (&w)[NW], const f16* p) {
  struct Words {
    uint32_t v[NW];
  } t;
  __builtin_memcpy(&t, p, sizeof(t));
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = t.v[i];
}

// Pair (row, kv head) of the next pass's layer-0 attention in the register form, one wave, for
// the sampled token tok: q of the pair's G heads and the new slot's k and v from the token's
// precomputed row (zeros if no index won), k and v into cache slot p and into the slot
// registers, then short_attn_wave over slots 0 .. p into o.
template <int HD, int G>
__device__ __forceinline__ void next_attention_reg(const NextPass& nx, int tok, int V, int row,
                                                   int kh, long cache, int lane,
                                                   NxvSlots<HD>& sl) {
  constexpr int NW = HD / 128, DPL = HD / 64;
  const int p = nx.p;
  const bool valid = (uint32_t)tok < (uint32_t)V;
  const f16* src = nx.qkv + (long)(valid ? tok : 0) * nx.qkv_ld + DPL * lane;
  uint32_t qw[G][NW], kn[NW], vn[NW];
  const uint32_t* ks = (const uint32_t*)(src + (long)(nx.Hq + kh) * HD);
  const uint32_t* vs = (const uint32_t*)(src + (long)(nx.Hq + nx.Hk + kh) * HD);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      qw[g][w] = valid ? ((const uint32_t*)(src + (long)(kh * G + g) * HD))[w] : 0u;
    kn[w] = valid ? ks[w] : 0u;
    vn[w] = valid ? vs[w] : 0u;
  }
  uint32_t* kd = (uint32_t*)(nx.kc + cache + (long)p * HD + DPL * lane);
  uint32_t* vd = (uint32_t*)(nx.vc + cache + (long)p * HD + DPL * lane);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    kd[w] = kn[w];
    vd[w] = vn[w];
  }
  // slot p takes the token's k and v: selects on values (a store at index p would move the
  // slot registers to scratch memory)
  uint32_t kw[NXV_SLOTS][NW], vw[NXV_SLOTS][NW];
#pragma unroll
  for (int t = 0; t < NXV_SLOTS; ++t)
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      kw[t][w] = t == p ? kn[w] : sl.k[t][w];
      vw[t][w] = t == p ? vn[w] : sl.v[t][w];
    }
  short_attn_wave<HD, G, NXV_SLOTS>(kw, vw, qw, p + 1, nx.scale,
                                    nx.o + (long)row * nx.o_ld + (long)kh * G * HD + DPL * lane);
}

// XHD: head_dim of the folded layer-0 attention (128: LDS form, 384: register form); the
// sampler alone (no qkv) runs the 128 instance.
template <int XHD>
__global__ __launch_bounds__(SMP_THREADS) void sample_topk_kernel(
    const f16* __restrict__ logits, long ld, int N, int cfg_on, float cfg, float temp, int topk,
    int V, const float* __restrict__ noise, const int64_t* __restrict__ seed,
    const int64_t* __restrict__ pos, int salt, int64_t* __restrict__ out, long out_stride,
    const NextPass nx) {
  __shared__ uint32_t hist[2][256];
  __shared__ uint32_t sel[4];  // threshold key, kept count; radix state
  __shared__ __align__(16) uint32_t wtot[SMP_THREADS / 64];
  __shared__ __align__(16) uint32_t wbin[SMP_WBINS_LDS];
  __shared__ int kept_i[SMP_MAXV];
  __shared__ float kept_x[SMP_MAXV];
  static_assert(XHD == NXA_HD || XHD == NXV_HD, "folded attention: head_dim 128 or 384");
  constexpr int AP = XHD == NXA_HD ? NXA_PAIRS : 1;  // the LDS form's arrays
  __shared__ __align__(16) f16 a_k[AP][NXA_SLOTS][NXA_HD];
  __shared__ __align__(16) f16 a_v[AP][NXA_SLOTS][NXA_HD];
  __shared__ __align__(16) f16 a_q[AP][NXA_G][NXA_HD];
  __shared__ float a_pe[AP][NXA_G][NXA_SLOTS];
  __shared__ int s_tok;

  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const f16* lc = logits + (long)n * ld;
  const f16* lu = logits + (long)(n + N) * ld;

  // 1. loads, all issued before any arithmetic: thread tid owns indices 8 tid .. 8 tid + 7
  //    (16-byte loads where the row stride allows) and 8192 + tid of the tail.  The Philox key
  //    and counter words are read here too, so their latency hides under the logits loads.
  const bool vec = ((ld & 7) == 0) && ((((uintptr_t)logits) & 15) == 0);
  const int i0 = 8 * tid;
  f16x8 c8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0}, u8 = c8;
  if (vec && i0 + 7 < V) {
    c8 = *(const f16x8*)(lc + i0);
    if (cfg_on) u8 = *(const f16x8*)(lu + i0);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (i0 + e < V) {
        c8[e] = lc[i0 + e];
        if (cfg_on) u8[e] = lu[i0 + e];
      }
  }
  const int it = 8 * SMP_THREADS + tid;
  f16 ct = (f16)0.0f, ut = ct;
  if (it < V) {
    ct = lc[it];
    if (cfg_on) ut = lu[it];
  }
  uint64_t sd = 0u, p64 = 0u;
  if (!noise) {  // seed and pos are only dereferenced on the Philox path (NULL with noise)
    sd = (uint64_t)seed[0];
    p64 = (uint64_t)pos[0];
  }
  // the next pass's layer-0 attention: wave 1 + j runs pair j (row n + (j / Hk) N, kv head
  // j % Hk); its cached slots 0 .. p - 1 (K and V) are loaded now: head_dim 128 into LDS (LDS
  // DMA, 4 slots per instruction, lanes past slot p - 1 idle), 384 into registers
  const int npairs = nx.qkv ? (cfg_on ? 2 : 1) * nx.Hk : 0;
  const int aj = wv - 1;
  const int arow = n + (aj / max(nx.Hk, 1)) * N, akh = aj - (aj / max(nx.Hk, 1)) * nx.Hk;
  const long acache = ((long)arow * nx.Hk + akh) * nx.L * XHD;  // the pair's [L, XHD] rows
  NxvSlots<XHD == NXV_HD ? NXV_HD : 128> sl;
  if constexpr (XHD == NXA_HD) {
    if (aj >= 0 && aj < npairs) {
      for (int u = 0; 4 * u < nx.p; ++u) {
        const int t = 4 * u + (lane >> 4);
        if (t < nx.p) {
          const uint32_t off = (uint32_t)(((long)t * NXA_HD + 8 * (lane & 15)) * 2);
          lds_dma16(nx.kc + acache, off, &a_k[aj][4 * u][0]);
          lds_dma16(nx.vc + acache, off, &a_v[aj][4 * u][0]);
        }
      }
    }
  }

  // 2. CFG mix in fp16, keys, and the block's largest key
  f16 lv[SMP_PER];
  uint32_t key[SMP_PER];
  uint32_t kmx = 0u;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    f16 l = j < 8 ? c8[j] : ct;
    if (cfg_on) {
      const f16 u = j < 8 ? u8[j] : ut;
      const f16 d = l - u;
      const f16 m = (f16)((float)d * cfg);
      l = u + m;
    }
    l = l + (f16)0.0f;  // -0.0 -> +0.0
    lv[j] = l;
    key[j] = (slot_index(tid, j) < V) ? hkey(l) : 0u;  // key 0: no value (hkey(x) > 0)
    kmx = max(kmx, key[j]);
  }
  kmx = wave_max_u32(kmx);
  if constexpr (XHD == NXV_HD) {
    // register form: the cached slots, once this wave's logits are in (issued earlier they would
    // queue ahead of the block's logits loads).  Every slot register is loaded, from slot
    // min(t, p - 1) (slot 0 when p = 0): no branch, so all the loads are in flight together;
    // slot p takes the token's k and v later and the slots past it are masked.
    constexpr int NW = XHD / 128;
    if (aj >= 0 && aj < npairs) {
      const f16* kb = nx.kc + acache + (XHD / 64) * lane;
      const f16* vb = nx.vc + acache + (XHD / 64) * lane;
      const int last = nx.p > 0 ? nx.p - 1 : 0;
#pragma unroll
      for (int t = 0; t < NXV_SLOTS; ++t) {
        ld_words<NW>(sl.k[t], kb + (long)min(t, last) * XHD);
        ld_words<NW>(sl.v[t], vb + (long)min(t, last) * XHD);
      }
    } else {
#pragma unroll
      for (int t = 0; t < NXV_SLOTS; ++t)
#pragma unroll
        for (int w = 0; w < NW; ++w) sl.k[t][w] = sl.v[t][w] = 0u;
    }
  }
  if (lane == 0) wtot[wv] = kmx;
  for (int b = tid; b < SMP_WBINS_LDS / 4; b += SMP_THREADS)
    ((u32x4*)wbin)[b] = (u32x4){0u, 0u, 0u, 0u};
  __syncthreads();

  // 3. histogram of the exact keys within SMP_WDIG digits below the largest one
  uint32_t kmax = 0u;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) kmax = max(kmax, wtot[w]);
  const uint32_t dtop = kmax >> 8;
  const uint32_t kbase = dtop >= SMP_WDIG - 1 ? (dtop - (SMP_WDIG - 1)) << 8 : 0u;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j)
    if (key[j] && key[j] >= kbase) atomicAdd(&wbin[wbin_at(key[j] - kbase)], 1u);
  __syncthreads();

  // 4. the walk from the top, by all threads: thread t owns the 4 window bins 4 (1023 - t) .. +3
  //    (thread 0 the top ones) as one 16-byte LDS word, and a block-wide scan of their counts
  //    from the top gives every bin's running count.  The threshold is the key at which the
  //    running count reaches k; every bin at or above it is replaced by the first kept slot of
  //    its key (kept values are stored in descending key order).
  static_assert(SMP_WBINS == 4 * SMP_THREADS, "four window bins per thread");
  const int b4 = 4 * (SMP_THREADS - 1 - tid);
  u32x4* const mine = (u32x4*)(wbin + wbin_at((uint32_t)b4));
  const u32x4 v = *mine;
  const uint32_t c = (v.x + v.y) + (v.z + v.w);
  const uint32_t winc = wave_incl_add_u32(c);
  if (lane == 63) wtot[wv] = winc;  // every thread read kmax from wtot before the last barrier
  __syncthreads();
  uint32_t before = 0u, wtotal = 0u;
#pragma unroll
  for (int w4 = 0; w4 < SMP_THREADS / 256; ++w4) {
    const u32x4 t = ((const u32x4*)wtot)[w4];
    const uint32_t tw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      before += 4 * w4 + r < wv ? tw[r] : 0u;
      wtotal += tw[r];
    }
  }
  const uint32_t k = (uint32_t)topk;
  const bool window = wtotal >= k;  // otherwise the radix select over all keys
  const uint32_t excl = before + winc - c;
  if (window && excl < k) {
    // running counts after each bin, from the top one (w) down
    const uint32_t a1 = excl + v.w, a2 = a1 + v.z, a3 = a2 + v.y, a4 = a3 + v.x;
    *mine = (u32x4){a3, a2, a1, excl};
    if (a4 >= k) {  // the thread holding the crossing
      const uint32_t below = (a1 < k ? 1u : 0u) + (a2 < k ? 1u : 0u) + (a3 < k ? 1u : 0u);
      sel[0] = kbase + (uint32_t)(b4 + 3) - below;
      sel[1] = below == 0u ? a1 : below == 1u ? a2 : below == 2u ? a3 : a4;
    }
  }
  __syncthreads();

  uint32_t total;
  if (window) {
    // 5. kept values (key >= threshold) to their slots; values with equal keys are equal, so
    //    their order among themselves does not change any sum below.  All the slot atomics are
    //    issued before the first store waits for one.
    const uint32_t thr = sel[0];
    total = sel[1];
    uint32_t slot[SMP_PER];
#pragma unroll
    for (int j = 0; j < SMP_PER; ++j)
      if (key[j] && key[j] >= thr) slot[j] = atomicAdd(&wbin[wbin_at(key[j] - kbase)], 1u);
#pragma unroll
    for (int j = 0; j < SMP_PER; ++j) {
      if (key[j] && key[j] >= thr) {
        kept_i[slot[j]] = slot_index(tid, j);
        kept_x[slot[j]] = (float)lv[j] / temp;
      }
    }
  } else {
    total = select_full(key, lv, temp, topk, hist, sel, wtot, kept_i, kept_x);
  }
  __syncthreads();
  if (wv != 0) {
    if (wv == SMP_THREADS / 64 - 1 && nx.ev) {  // the last wave: rows n (and n + N) of ev
      for (int h = 0; h < 1 + cfg_on; ++h) {
        f16x8 v[SMP_RCH];
        row_load(v, nx.ev + (long)(n + h * N) * nx.ev_ld, nx.D, true, lane);
        row_store(v, nx.xe + (long)(n + h * N) * nx.xe_ld, nullptr, nx.D, lane);
      }
    }
    if (aj < npairs) {  // a pair wave: the token, then the pair's attention
      __syncthreads();
      if constexpr (XHD == NXA_HD) {
        next_attention(nx, s_tok, V, aj, arow, akh, acache, lane, a_k[aj], a_v[aj], a_q[aj],
                       a_pe[aj]);
      } else {
        next_attention_reg<XHD, NXV_G>(nx, s_tok, V, arow, akh, acache, lane, sl);
      }
    }
    return;
  }

  // 6. wave 0: log_softmax then softmax in fp32 over the kept values (app/engine.py:293-296);
  //    the largest x is the one of the largest key
  const float m1 = (float)hkey_inv(kmax) / temp;
  float s1 = 0.f;
  for (uint32_t b = lane; b < total; b += 64) s1 += expf(kept_x[b] - m1);
  s1 = wave_sum_dpp(s1);
  const float logsum = logf(s1);
  // the maximum of ls = (x - m1) - logsum is exactly -logsum (at x = m1)
  const float m2 = 0.f - logsum;
  float s2 = 0.f;
  for (uint32_t b = lane; b < total; b += 64) s2 += expf(((kept_x[b] - m1) - logsum) - m2);
  s2 = wave_sum_dpp(s2);

  // 7. exponential race: argmax p / q, q ~ Exp(1); draws for index i come from Philox block
  //    (i / 4, take, pos, salt), word i % 4 (or the injected noise)
  const uint32_t k0 = (uint32_t)sd, k1 = (uint32_t)(sd >> 32);
  float bv = -1.f;
  int bi = 0x7FFFFFFF;
  for (uint32_t b = lane; b < total; b += 64) {
    const int i = kept_i[b];
    float q;
    if (noise) {
      q = noise[(long)n * V + i];
    } else {
      uint32_t c[4] = {(uint32_t)(i >> 2), (uint32_t)n, (uint32_t)p64,
                       (uint32_t)(p64 >> 32) ^ ((uint32_t)salt << 20)};
      philox4x32_10(c, k0, k1);
      const uint32_t w = c[i & 3];
      const float u = ((float)(w >> 8) + 0.5f) * (1.0f / 16777216.0f);
      q = -logf(u);
    }
    const float p = expf(((kept_x[b] - m1) - logsum) - m2) / s2;
    const float r = p / q;
    if (r > bv || (r == bv && i < bi)) {
      bv = r;
      bi = i;
    }
  }
  // wave argmax, lowest index on ties: r >= 0 (or no candidate in the lane), so the bit
  // patterns order like the values
  const uint32_t rb = bi == 0x7FFFFFFF ? 0u : __builtin_bit_cast(uint32_t, bv);
  const uint32_t mb = wave_max_u32(rb);
  bi = (int)wave_min_u32(rb == mb ? (uint32_t)bi : 0xFFFFFFFFu);
  if (npairs) {  // the token to the pair waves
    if (lane == 0) s_tok = bi;
    __syncthreads();
  }
  if (lane == 0) {
    out[(long)n * out_stride] = bi;
    if (cfg_on) out[(long)(n + N) * out_stride] = bi;
  }
  // 8. the next pass's input row of the sampled token (rows [V, D] precomputed from it) into
  //    x rows n and n + N; zeros if no index won (NaN logits)
  if (nx.rows) {
    const bool valid = (uint32_t)bi < (uint32_t)V;
    f16x8 v[SMP_RCH];
    row_load(v, nx.rows + (long)(valid ? bi : 0) * nx.rows_ld, nx.D, valid, lane);
    row_store(v, nx.x + (long)n * nx.x_ld, cfg_on ? nx.x + (long)(n + N) * nx.x_ld : nullptr,
              nx.D, lane);
  }
}

// ---------------------------------------------------------------- end of a frame
// Frame bookkeeping of the song loop kept on the device, so a captured frame needs no host
// work between replays (the host only reads first_eos every few frames): the frame's tokens
// become the next frame's input, rows 0..N-1 are stored as frame f = pos - P + 1 of the song,
// each take's first frame holding a token >= eos is recorded (frames 1..F only: the frame of
// the prompt pass is never scanned, as in app/engine.py:433-437), and the position advances.
// One block; thread i handles token (i / 8, i % 8) of the B x 8 frame.
__global__ __launch_bounds__(512) void frame_advance_kernel(
    const int64_t* __restrict__ samples, long lds, int64_t* __restrict__ tok, long ldt,
    int64_t* __restrict__ pos, long ldp, int64_t* __restrict__ out,
    int64_t* __restrict__ first_eos, int B, int N, int P, int F, int64_t eos) {
  __shared__ int hit[64];
  const int i = threadIdx.x;
  const int b = i >> 3, c = i & 7;
  const long f = pos[0] - (long)P + 1;  // every row holds the same position
  if (i < 64) hit[i] = 0;
  __syncthreads();
  if (b < B) {
    const int64_t t = samples[(long)b * lds + c];
    tok[(long)b * ldt + c] = t;
    if (b < N && f >= 0 && f <= F) out[(f * N + b) * 8 + c] = t;
    if (b < N && t >= eos) hit[b] = 1;
  }
  __syncthreads();  // every thread has read pos before it moves
  if (i < N && hit[i] && f >= 1 && f <= F && first_eos[i] < 0) first_eos[i] = f;
  if (i < B) pos[(long)i * ldp] += 1;
}

}  // namespace ecd

using namespace ecd;

extern "C" int ecd_frame_advance(const int64_t* samples, long lds, int64_t* tok, long ldt,
                                 int64_t* pos, long ldp, int64_t* out, int64_t* first_eos, int B,
                                 int N, int P, int F, int64_t eos, void* stream) {
  if (!samples || !tok || !pos || !out || !first_eos || B <= 0 || B > 64 || N <= 0 || N > B ||
      lds < 8 || ldt < 8 || ldp < 1 || F < 0 || P < 0)
    return ECD_EINVAL;
  hipLaunchKernelGGL(frame_advance_kernel, dim3(1), dim3(B * 8), 0, (hipStream_t)stream, samples,
                     lds, tok, ldt, pos, ldp, out, first_eos, B, N, P, F, eos);
  return ecd_launch_status();
}

extern "C" int ecd_sample_topk(const void* logits, long ld, int B, int N, float cfg, float temp,
                               int topk, int V, const float* noise, const int64_t* seed,
                               const int64_t* pos, int salt, int64_t* out, long out_stride,
                               void* stream) {
  if (!logits || !out || N <= 0 || V <= 0 || V > SMP_MAXV || ld < V || topk <= 0 || topk > V ||
      !(temp > 0.f) || out_stride <= 0 || (B != N && B != 2 * N) ||
      (!noise && (!seed || !pos)))
    return ECD_EINVAL;
  const int cfg_on = (B == 2 * N) ? 1 : 0;
  hipLaunchKernelGGL(sample_topk_kernel<NXA_HD>, dim3(N), dim3(SMP_THREADS), 0,
                     (hipStream_t)stream, (const f16*)logits, ld, N, cfg_on, cfg, temp, topk, V,
                     noise, seed, pos, salt, out, out_stride, NextPass{});
  return ecd_launch_status();
}

extern "C" int ecd_sample_topk_next(const void* logits, long ld, int B, int N, float cfg,
                                    float temp, int topk, int V, const float* noise,
                                    const int64_t* seed, const int64_t* pos, int salt,
                                    int64_t* out, long out_stride, const void* rows, long rows_ld,
                                    int rows_n, void* x, long x_ld, int D, const void* qkv,
                                    long qkv_ld, int qkv_n, void* kc, void* vc, int L, int p,
                                    void* o, long o_ld, int Hq, int Hk, int HD,
                                    const void* ev, long ev_ld, void* xe, long xe_ld,
                                    void* stream) {
  const auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  if (!rows || !x || rows_n < V || D <= 0 || D > 512 * SMP_RCH || (D % 8) || rows_ld < D ||
      (rows_ld % 8) ||
      x_ld < D || (x_ld % 8) || !al(rows) || !al(x))
    return ECD_EINVAL;
  if (!logits || !out || N <= 0 || V <= 0 || V > SMP_MAXV || ld < V || topk <= 0 || topk > V ||
      !(temp > 0.f) || out_stride <= 0 || (B != N && B != 2 * N) ||
      (!noise && (!seed || !pos)))
    return ECD_EINVAL;
  const int cfg_on = B == 2 * N ? 1 : 0;
  if (qkv) {
    const bool lds_form = HD == NXA_HD;
    if (!lds_form && HD != NXV_HD) return ECD_EINVAL;
    const int nq = (Hq + 2 * Hk) * HD;
    if (!kc || !vc || !o || Hk <= 0 || Hq <= 0 || (Hq % Hk) ||
        (lds_form ? Hq / Hk > NXA_G : Hq / Hk != NXV_G) ||
        (1 + cfg_on) * Hk > (lds_form ? NXA_PAIRS : NXV_PAIRS) || p < 0 || p >= L ||
        p >= (lds_form ? NXA_SLOTS : NXV_SLOTS) || qkv_n < V || qkv_ld < nq || (qkv_ld % 8) ||
        o_ld < Hq * HD || (o_ld % 8) || !al(qkv) || !al(kc) || !al(vc) || !al(o))
      return ECD_EINVAL;
  }
  if (ev && (!xe || ev_ld < D || (ev_ld % 8) || xe_ld < D || (xe_ld % 8) || !al(ev) || !al(xe)))
    return ECD_EINVAL;
  NextPass nx{};
  nx.ev = (const f16*)ev; nx.ev_ld = ev_ld; nx.xe = (f16*)xe; nx.xe_ld = xe_ld;
  nx.rows = (const f16*)rows; nx.rows_ld = rows_ld; nx.x = (f16*)x; nx.x_ld = x_ld; nx.D = D;
  if (qkv) {
    nx.qkv = (const f16*)qkv; nx.qkv_ld = qkv_ld; nx.kc = (f16*)kc; nx.vc = (f16*)vc;
    nx.L = L; nx.p = p; nx.o = (f16*)o; nx.o_ld = o_ld; nx.Hq = Hq; nx.Hk = Hk; nx.HD = HD;
    nx.scale = (float)(1.0 / sqrt((double)HD));  // the fp32 rounding of 1 / sqrt(HD)
  }
  if (qkv && HD == NXV_HD)
    hipLaunchKernelGGL(sample_topk_kernel<NXV_HD>, dim3(N), dim3(SMP_THREADS), 0,
                       (hipStream_t)stream, (const f16*)logits, ld, N, cfg_on, cfg, temp, topk, V,
                       noise, seed, pos, salt, out, out_stride, nx);
  else
    hipLaunchKernelGGL(sample_topk_kernel<NXA_HD>, dim3(N), dim3(SMP_THREADS), 0,
                       (hipStream_t)stream, (const f16*)logits, ld, N, cfg_on, cfg, temp, topk, V,
                       noise, seed, pos, salt, out, out_stride, nx);
  return ecd_launch_status();
}
