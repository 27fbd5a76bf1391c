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
// One block of 1024 threads per take.  The k-th largest value comes from a two-pass radix select
// (8-bit digits, LDS histograms) on order-preserving 16-bit keys of the fp16 logits: x =
// fp32(l)/temp is strictly monotonic in l, so the threshold and its ties are those of l.  Only
// the kept values (key >= threshold, k of them plus ties) reach the softmax and the race:
// every other index has p = 0 exactly and can neither win nor change a sum.  The kept values
// are compacted into LDS in (thread, slot) order by prefix sums, so their fp32 sums are formed
// in a fixed order, and one wave finishes the softmax and the race without further barriers.
// The Exponential(1) draws are q = -log(u), u = (bits >> 8 + 0.5) * 2^-24 from the
// counter-based Philox4x32-10 generator (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011), keyed by a 64-bit seed read from device memory and
// countered by (vocab index / 4, take, frame position, salt): graph replays at different
// frame positions draw fresh numbers without any mutable RNG state.  Tests can inject the
// draws instead (noise [N, V] fp32).
#include "common.h"

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
constexpr int SMP_MAXV = 8704;  // LDS capacity in values (8197 codebook entries + slack)

// Order-preserving 16-bit key of an fp16 value (-0.0 must be canonicalised to +0.0 first so
// that key order equals float comparison).
__device__ __forceinline__ uint32_t hkey(f16 h) {
  const uint32_t u = __builtin_bit_cast(uint16_t, h);
  return (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
}

constexpr int SMP_GRP = (SMP_MAXV + 8 * SMP_THREADS - 1) / (8 * SMP_THREADS);  // 8-value groups
constexpr int SMP_PER = 8 * SMP_GRP;  // values per thread

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

__global__ __launch_bounds__(SMP_THREADS) void sample_topk_kernel(
    const f16* __restrict__ logits, long ld, int N, int cfg_on, float cfg, float temp, int topk,
    int V, const float* __restrict__ noise, const int64_t* __restrict__ seed,
    const int64_t* __restrict__ pos, int salt, int64_t* __restrict__ out, long out_stride) {
  __shared__ uint32_t hist[2][256];
  __shared__ uint32_t sel[2];  // selected key prefix, remaining rank
  __shared__ uint32_t wtot[SMP_THREADS / 64];
  __shared__ int kept_i[SMP_MAXV];
  __shared__ float kept_x[SMP_MAXV];

  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const f16* lc = logits + (long)n * ld;
  const f16* lu = logits + (long)(n + N) * ld;

  // 1. CFG mix in fp16.  Thread tid owns indices 8 tid + e + 8192 g (e < 8, g < SMP_GRP): the
  //    loads are 16 bytes per lane where the row stride allows it.
  f16 lv[SMP_PER];
  uint32_t key[SMP_PER];
  const bool vec = ((ld & 7) == 0) && ((((uintptr_t)logits) & 15) == 0);
#pragma unroll
  for (int g = 0; g < SMP_GRP; ++g) {
    const int i0 = 8 * tid + SMP_THREADS * 8 * g;
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
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = 8 * g + e;
      f16 l = c8[e];
      if (cfg_on) {
        const f16 d = l - u8[e];
        const f16 m = (f16)((float)d * cfg);
        l = u8[e] + m;
      }
      l = l + (f16)0.0f;  // -0.0 -> +0.0
      lv[j] = l;
      key[j] = (i0 + e < V) ? hkey(l) : 0u;
    }
  }
  if (tid < 256) {
    hist[0][tid] = 0u;
    hist[1][tid] = 0u;
  }
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = (uint32_t)topk;
  }
  __syncthreads();

  // 2. k-th largest fp16 value by a two-pass radix select on the 16-bit keys (key 0 marks an
  //    index past V: hkey is nonzero for every fp16 value except the NaN pattern 0xFFFF)
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

  // 3. compact the kept indices (key >= thr) in (thread, slot) order: a wave-level inclusive
  //    scan of per-thread counts, then per-wave totals through LDS
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
      kept_i[base] = 8 * tid + (j & 7) + SMP_THREADS * 8 * (j >> 3);
      kept_x[base] = (float)lv[j] / temp;
      ++base;
    }
  }
  __syncthreads();
  if (wv != 0) return;

  // 4. wave 0: log_softmax then softmax in fp32 over the kept values (app/engine.py:293-296)
  float m1 = -INFINITY;
  for (int b = lane; b < total; b += 64) m1 = fmaxf(m1, kept_x[b]);
  m1 = wave_max(m1);
  float s1 = 0.f;
  for (int b = lane; b < total; b += 64) s1 += expf(kept_x[b] - m1);
  s1 = wave_sum(s1);
  const float logsum = logf(s1);
  // the maximum of ls = (x - m1) - logsum is exactly -logsum (at x = m1)
  const float m2 = 0.f - logsum;
  float s2 = 0.f;
  for (int b = lane; b < total; b += 64) s2 += expf(((kept_x[b] - m1) - logsum) - m2);
  s2 = wave_sum(s2);

  // 5. exponential race: argmax p / q, q ~ Exp(1); draws for index i come from Philox block
  //    (i / 4, take, pos, salt), word i % 4 (or the injected noise)
  uint32_t k0 = 0u, k1 = 0u;
  uint64_t p64 = 0u;
  if (!noise) {  // seed and pos are only dereferenced on the Philox path (NULL with noise)
    const uint64_t sd = (uint64_t)seed[0];
    k0 = (uint32_t)sd;
    k1 = (uint32_t)(sd >> 32);
    p64 = (uint64_t)pos[0];
  }
  float bv = -1.f;
  int bi = 0x7FFFFFFF;
  for (int b = lane; b < total; b += 64) {
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
  // wave argmax, lowest index on ties
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    out[(long)n * out_stride] = bi;
    if (cfg_on) out[(long)(n + N) * out_stride] = bi;
  }
}

}  // namespace ecd

using namespace ecd;

extern "C" int ecd_sample_topk(const void* logits, long ld, int B, int N, float cfg, float temp,
                               int topk, int V, const float* noise, const int64_t* seed,
                               const int64_t* pos, int salt, int64_t* out, long out_stride,
                               void* stream) {
  if (!logits || !out || N <= 0 || V <= 0 || V > SMP_MAXV || ld < V || topk <= 0 || topk > V ||
      !(temp > 0.f) || out_stride <= 0 || (B != N && B != 2 * N) ||
      (!noise && (!seed || !pos)))
    return ECD_EINVAL;
  const int cfg_on = (B == 2 * N) ? 1 : 0;
  hipLaunchKernelGGL(sample_topk_kernel, dim3(N), dim3(SMP_THREADS), 0, (hipStream_t)stream,
                     (const f16*)logits, ld, N, cfg_on, cfg, temp, topk, V, noise, seed, pos, salt,
                     out, out_stride);
  return ecd_launch_status();
}
