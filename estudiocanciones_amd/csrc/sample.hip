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

// Order-preserving 16-bit key of an fp16 value (-0.0 must be canonicalised to +0.0 first so
// that key order equals float comparison).
__device__ __forceinline__ uint32_t hkey(f16 h) {
  const uint32_t u = __builtin_bit_cast(uint16_t, h);
  return (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
}

constexpr int SMP_PER = (SMP_MAXV + SMP_THREADS - 1) / SMP_THREADS;  // values per thread

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
  __shared__ float red[SMP_THREADS / 64];
  __shared__ uint32_t sel[2];  // selected key prefix, remaining rank
  __shared__ float bestv[SMP_THREADS / 64];
  __shared__ int besti[SMP_THREADS / 64];

  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const f16* lc = logits + (long)n * ld;
  const f16* lu = logits + (long)(n + N) * ld;

  // 1. CFG mix in fp16 (values stay in registers: thread tid owns indices tid + 1024 j)
  f16 lv[SMP_PER];
  uint32_t key[SMP_PER];
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    const int i = tid + SMP_THREADS * j;
    key[j] = 0u;
    lv[j] = (f16)0.0f;
    if (i < V) {
      f16 l = lc[i];
      if (cfg_on) {
        const f16 u = lu[i];
        const f16 d = l - u;
        const f16 e = (f16)((float)d * cfg);
        l = u + e;
      }
      l = l + (f16)0.0f;  // -0.0 -> +0.0
      lv[j] = l;
      key[j] = hkey(l);
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

  // 2. k-th largest fp16 value by a two-pass radix select on the 16-bit keys.  x = fp32(l)/temp
  //    is strictly monotonic in l, so the threshold and the ties of the reference's fp32 topk
  //    are those of l.
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j)
    if (tid + SMP_THREADS * j < V) atomicAdd(&hist[0][key[j] >> 8], 1u);
  __syncthreads();
  if (tid < 64) radix_pick(hist[0], sel, 0u, 8, lane);
  __syncthreads();
  const uint32_t hi8 = sel[0];
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j)
    if (tid + SMP_THREADS * j < V && (key[j] & 0xFF00u) == hi8) atomicAdd(&hist[1][key[j] & 255u], 1u);
  __syncthreads();
  if (tid < 64) radix_pick(hist[1], sel, hi8, 0, lane);
  __syncthreads();
  const uint32_t thr = sel[0];

  // 3. masked logits / temp; log_softmax then softmax in fp32 (app/engine.py:293-296)
  float xv[SMP_PER];
  float mloc = -INFINITY;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    const bool in = tid + SMP_THREADS * j < V && key[j] >= thr;
    xv[j] = in ? (float)lv[j] / temp : -INFINITY;
    mloc = fmaxf(mloc, xv[j]);
  }
  const float m1 = block_reduce_max(mloc, red);
  float sloc = 0.f;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) sloc += expf(xv[j] - m1);
  const float s1 = block_reduce_sum(sloc, red);
  const float logsum = logf(s1);
  // the maximum of ls = (x - m1) - logsum is exactly -logsum (at x = m1)
  const float m2 = 0.f - logsum;
  float s2loc = 0.f;
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    xv[j] = (xv[j] - m1) - logsum;
    s2loc += expf(xv[j] - m2);
  }
  const float s2 = block_reduce_sum(s2loc, red);

  // 4. exponential race: argmax p / q, q ~ Exp(1); draws for index i come from Philox block
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
#pragma unroll
  for (int j = 0; j < SMP_PER; ++j) {
    const int i = tid + SMP_THREADS * j;
    if (i < V) {
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
      const float p = expf(xv[j] - m2) / s2;
      const float r = p / q;
      if (r > bv || (r == bv && i < bi)) {
        bv = r;
        bi = i;
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
  if (lane == 0) {
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
