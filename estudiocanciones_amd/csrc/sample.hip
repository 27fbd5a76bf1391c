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
// One block of 1024 threads per take.  The k-th largest value is found by an exact 4-pass
// radix select (8-bit digits) on order-preserving uint32 keys of the fp32 values in LDS.
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

// Order-preserving key: larger float -> larger unsigned key (finite and -inf values).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float keyf(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __builtin_bit_cast(float, u);
}

constexpr int SMP_THREADS = 1024;
constexpr int SMP_MAXV = 8704;  // LDS capacity in values (8197 codebook entries + slack)

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < SMP_THREADS / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < SMP_THREADS / 64; ++i) r += red[i];
  return r;
}

__global__ __launch_bounds__(SMP_THREADS) void sample_topk_kernel(
    const f16* __restrict__ logits, long ld, int N, int cfg_on, float cfg, float temp, int topk,
    int V, const float* __restrict__ noise, const int64_t* __restrict__ seed,
    const int64_t* __restrict__ pos, int salt, int64_t* __restrict__ out, long out_stride) {
  __shared__ float xs[SMP_MAXV];
  __shared__ uint32_t hist[256];
  __shared__ float red[SMP_THREADS / 64];
  __shared__ uint32_t sel[2];  // selected prefix, remaining rank
  __shared__ float bestv[SMP_THREADS / 64];
  __shared__ int besti[SMP_THREADS / 64];

  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const f16* lc = logits + (long)n * ld;
  const f16* lu = logits + (long)(n + N) * ld;

  // 1. CFG mix in fp16, temperature in fp32
  for (int i = tid; i < V; i += SMP_THREADS) {
    f16 l = lc[i];
    if (cfg_on) {
      const f16 u = lu[i];
      const f16 d = l - u;
      const f16 e = (f16)((float)d * cfg);
      l = u + e;
    }
    xs[i] = (float)l / temp;
  }
  __syncthreads();

  // 2. exact k-th largest value by radix select on the keys
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = (uint32_t)topk;
  }
  uint32_t mask = 0u;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
    const uint32_t prefix = sel[0];
    for (int base = 0; base < V; base += SMP_THREADS) {
      const int i = base + tid;
      bool act = false;
      uint32_t dg = 0u;
      if (i < V) {
        const uint32_t k = fkey(xs[i]);
        act = (k & mask) == prefix;
        dg = (k >> shift) & 255u;
      }
      // few distinct digits dominate (the top byte of the keys especially): count up to four
      // of them per wave with one LDS atomic each, the rest with per-lane atomics
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const uint64_t pend = __ballot(act);
        if (pend == 0) break;
        const int leader = __ffsll((unsigned long long)pend) - 1;
        const uint32_t d0 = __shfl(dg, leader, 64);
        const uint64_t same = __ballot(act && dg == d0);
        if ((tid & 63) == leader) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
        if (dg == d0) act = false;
      }
      if (act) atomicAdd(&hist[dg], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // find the digit (from the top) where the cumulative count reaches the rank
      const uint32_t rank = sel[1];
      // each lane sums 4 bins, counting down from digit 255
      uint32_t c4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) c4 += hist[255 - (tid * 4 + j)];
      // inclusive prefix over lanes (lane 0 = highest digits)
      uint32_t incl = c4;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, 64);
        if (tid >= o) incl += t;
      }
      const uint32_t excl = incl - c4;
      if (excl < rank && incl >= rank) {
        uint32_t acc = excl;
        for (int j = 0; j < 4; ++j) {
          const uint32_t d = 255 - (tid * 4 + j);
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
    __syncthreads();
    mask |= 255u << shift;
  }
  const float thr = keyf(sel[0]);

  // 3. mask below the threshold; log_softmax then softmax, fp32
  float mloc = -INFINITY;
  for (int i = tid; i < V; i += SMP_THREADS) {
    float x = xs[i];
    x = x < thr ? -INFINITY : x;
    xs[i] = x;
    mloc = fmaxf(mloc, x);
  }
  const float m1 = block_reduce_max(mloc, red);
  float sloc = 0.f;
  for (int i = tid; i < V; i += SMP_THREADS) sloc += expf(xs[i] - m1);
  const float s1 = block_reduce_sum(sloc, red);
  const float logsum = logf(s1);
  // log_softmax: ls = (x - m1) - logsum; its maximum is exactly -logsum (at x = m1, where
  // (m1 - m1) - logsum is exact), so the second softmax needs no max reduction
  const float m2 = 0.f - logsum;
  float s2loc = 0.f;
  for (int i = tid; i < V; i += SMP_THREADS) {
    const float ls = (xs[i] - m1) - logsum;
    xs[i] = ls;
    s2loc += expf(ls - m2);
  }
  const float s2 = block_reduce_sum(s2loc, red);

  // 4. exponential race
  // seed and pos are only dereferenced on the Philox path (they may be NULL with noise)
  uint32_t k0 = 0u, k1 = 0u;
  uint64_t p64 = 0u;
  if (!noise) {
    const uint64_t sd = (uint64_t)seed[0];
    k0 = (uint32_t)sd;
    k1 = (uint32_t)(sd >> 32);
    p64 = (uint64_t)pos[0];
  }
  float bv = -1.f;
  int bi = 0x7FFFFFFF;
  for (int base = tid * 4; base < V; base += SMP_THREADS * 4) {
    float q[4];
    if (noise) {
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = base + j < V ? noise[(long)n * V + base + j] : 1.f;
    } else {
      uint32_t c[4] = {(uint32_t)(base >> 2), (uint32_t)n, (uint32_t)p64,
                       (uint32_t)(p64 >> 32) ^ ((uint32_t)salt << 20)};
      philox4x32_10(c, k0, k1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float u = ((float)(c[j] >> 8) + 0.5f) * (1.0f / 16777216.0f);
        q[j] = -logf(u);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = base + j;
      if (i < V) {
        const float p = expf(xs[i] - m2) / s2;
        const float r = p / q[j];
        if (r > bv || (r == bv && i < bi)) {
          bv = r;
          bi = i;
        }
      }
    }
  }
  // block argmax, lowest index on ties
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    bestv[tid >> 6] = bv;
    besti[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = bestv[0];
    int ix = besti[0];
    for (int w = 1; w < SMP_THREADS / 64; ++w) {
      if (bestv[w] > v || (bestv[w] == v && besti[w] < ix)) {
        v = bestv[w];
        ix = besti[w];
      }
    }
    out[(long)n * out_stride] = ix;
    if (cfg_on) out[(long)(n + N) * out_stride] = ix;
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
