// Row-wise and element-wise kernels of the per-frame decode step (gfx950):
// RMSNorm, RoPE + KV-cache write, SiLU(a)*b, embedding gathers, the per-row
// int8 quantiser and the Llama-3-scaled RoPE table.  All fp16 rounding points follow
// the reference kernels (app/kernels.py) exactly; accumulation is fp32.
#include "common.h"

namespace ecd {

// ---------------------------------------------------------------- RMSNorm
// y = fp16( fp16(x * inv) * w ),  inv = 1 / sqrt(sum(x^2) / D + eps)   (app/kernels.py:58-67)
template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void rmsnorm_kernel(const f16* __restrict__ x, long ldx,
                                                        const f16* __restrict__ w,
                                                        f16* __restrict__ y, long ldy, int D,
                                                        float eps) {
  const f16* xr = x + (long)blockIdx.x * ldx;
  f16* yr = y + (long)blockIdx.x * ldy;
  float ss = 0.f;
  for (int i = threadIdx.x; i < D; i += BLOCK) {
    const float v = (float)xr[i];
    ss += v * v;
  }
  ss = wave_sum(ss);
  __shared__ float part[BLOCK / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < BLOCK / 64; ++i) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / (float)D + eps);
  for (int i = threadIdx.x; i < D; i += BLOCK) {
    const f16 h = (f16)((float)xr[i] * inv);
    yr[i] = h * w[i];
  }
}

// The same RMSNorm, one wave per row for D = 512 NV: each lane holds 8 NV elements (NV 16-byte
// loads), so the row is read once, and the sum of squares is one wave reduction (the fp32
// summation order differs from rmsnorm_kernel's; the rounding points do not).
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const f16* __restrict__ x, long ldx,
                                                           const f16* __restrict__ w,
                                                           f16* __restrict__ y, long ldy, int R,
                                                           float eps) {
  const int lane = threadIdx.x & 63;
  const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const f16x8* xr = (const f16x8*)(x + r * ldx);
  f16x8 v[NV], wv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = xr[lane + 64 * i];
#pragma unroll
  for (int i = 0; i < NV; ++i) wv[i] = ((const f16x8*)w)[lane + 64 * i];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = (float)v[i][e];
      ss += f * f;
    }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)(512 * NV) + eps);
  f16x8* yr = (f16x8*)(y + r * ldy);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (f16)((float)v[i][e] * inv);
    yr[lane + 64 * i] = h * wv[i];
  }
}

// ---------------------------------------------------------------- RoPE + KV-cache write
// One block per row r (batch b = r / S, position p = pos[r]).  Interleaved pairs
// (x[2i], x[2i+1]) are rotated by the table entry rope[p, i] = (cos, sin); q heads go to
// q_out, k heads to kc[b, kh, p, :], v heads are copied to vc[b, kh, p, :]
// (app/kernels.py:78-107).  A row whose position is outside [0, L) writes no cache slot
// and rotates q with the clamped position.
__global__ __launch_bounds__(256) void rope_kv_kernel(const f16* __restrict__ qkv,
                                                      const float* __restrict__ rope,
                                                      const int64_t* __restrict__ pos,
                                                      f16* __restrict__ q, f16* __restrict__ kc,
                                                      f16* __restrict__ vc, int S, int Hq, int Hk,
                                                      int L, int HD) {
  const int r = blockIdx.x;
  const int b = r / S;
  const long p_raw = pos[r];
  const bool pval = p_raw >= 0 && p_raw < L;
  const long p = p_raw < 0 ? 0 : (p_raw >= L ? L - 1 : p_raw);
  const int half = HD >> 1;
  const long W = (long)(Hq + 2 * Hk) * HD;
  const f16* src = qkv + (long)r * W;
  const float2* tab = (const float2*)(rope + p * HD);
  const int npairs = (Hq + Hk) * half;
  for (int i = threadIdx.x; i < npairs; i += 256) {
    const int h = i / half, j = i - h * half;
    const float2 cs = tab[j];
    const f16x2 xv = *(const f16x2*)(src + (long)h * HD + 2 * j);
    const float x0 = (float)xv.x, x1 = (float)xv.y;
    f16x2 o;
    o.x = (f16)(x0 * cs.x - x1 * cs.y);
    o.y = (f16)(x1 * cs.x + x0 * cs.y);
    if (h < Hq) {
      *(f16x2*)(q + (long)r * Hq * HD + (long)h * HD + 2 * j) = o;
    } else if (pval) {
      const int kh = h - Hq;
      *(f16x2*)(kc + (((long)b * Hk + kh) * L + p) * HD + 2 * j) = o;
    }
  }
  if (!pval) return;
  const f16* vs = src + (long)(Hq + Hk) * HD;
  const int nv = Hk * half;
  for (int i = threadIdx.x; i < nv; i += 256) {
    const int kh = i / half, j = i - kh * half;
    *(f16x2*)(vc + (((long)b * Hk + kh) * L + p) * HD + 2 * j) =
        *(const f16x2*)(vs + (long)kh * HD + 2 * j);
  }
}

// ---------------------------------------------------------------- SiLU(a) * b
// y[r, c] = fp16( fp16(silu_fp32(a)) * b ),  a = x[r, c], b = x[r, F + c]  (app/kernels.py:171-180)
__global__ __launch_bounds__(256) void silu_mul_kernel(const f16* __restrict__ x,
                                                       f16* __restrict__ y, int F) {
  const int r = blockIdx.y;
  const int c8 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c8 >= F) return;
  const f16* a = x + (long)r * 2 * F;
  const f16* bsrc = a + F;
  f16* yr = y + (long)r * F;
  if (c8 + 8 <= F && (F & 7) == 0) {
    const f16x8 av = *(const f16x8*)(a + c8);
    const f16x8 bv = *(const f16x8*)(bsrc + c8);
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float af = (float)av[e];
      const f16 sg = (f16)(af / (1.0f + expf(-af)));
      o[e] = sg * bv[e];
    }
    *(f16x8*)(yr + c8) = o;
  } else {
    for (int c = c8; c < min(c8 + 8, F); ++c) {
      const float af = (float)a[c];
      const f16 sg = (f16)(af / (1.0f + expf(-af)));
      yr[c] = sg * bsrc[c];
    }
  }
}

// ---------------------------------------------------------------- embeddings
// Tables are int8 rows with per-row fp16 scales (e = fp16(fp16(q[row]) * s[row]),
// app/engine.py:98) or, when no scales are given, dense fp16 rows (the bf16 tables of files
// written with --keep-emb-bf16, loaded as fp16: e = w[row], app/engine.py:95-97, :244-247).
__device__ __forceinline__ f16 emb_at(const void* table, const f16* scales, long rowi, long D,
                                      int d) {
  if (scales) return (f16)(float)((const int8_t*)table)[rowi * D + d] * scales[rowi];
  return ((const f16*)table)[rowi * D + d];
}

// Backbone input (app/engine.py:98, :348): out[b, :] = fp16( sum_c e(row) ), row = tok[b, c] +
// c * vocab, accumulated in fp32 over the C codebooks.  A token outside [0, vocab) (or a row
// beyond the table) contributes nothing.
__global__ __launch_bounds__(256) void embed_sum_kernel(const int64_t* __restrict__ tok,
                                                        const void* __restrict__ table,
                                                        const f16* __restrict__ scales,
                                                        f16* __restrict__ out, int C, int D,
                                                        int vocab, long rows) {
  const int b = blockIdx.y;
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= D) return;
  float acc = 0.f;
  for (int c = 0; c < C; ++c) {
    const long t = tok[(long)b * C + c];
    const long rowi = t + (long)c * vocab;
    if (t < 0 || t >= vocab || rowi >= rows) continue;
    acc += (float)emb_at(table, scales, rowi, D, d);
  }
  out[(long)b * D + d] = (f16)acc;
}

// Decoder input (app/engine.py:307-308, :336, :342): out[b] = e(row) with
// row = tok[b * tok_stride] + cb * vocab.  With `even` set, row 2b of out receives even[b]
// and row 2b+1 the embedding (the two-row interleave of the first decoder pass).
__global__ __launch_bounds__(256) void embed_one_kernel(const int64_t* __restrict__ tok,
                                                        long tok_stride,
                                                        const void* __restrict__ table,
                                                        const f16* __restrict__ scales, int cb,
                                                        int vocab, long rows,
                                                        const f16* __restrict__ even,
                                                        f16* __restrict__ out, int D) {
  const int b = blockIdx.y;
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= D) return;
  const long t = tok[(long)b * tok_stride];
  f16 e = (f16)0.0f;
  const long rowi = t + (long)cb * vocab;
  if (t >= 0 && t < vocab && rowi < rows) e = emb_at(table, scales, rowi, D, d);
  if (even) {
    out[(2L * b) * D + d] = even[(long)b * D + d];
    out[(2L * b + 1) * D + d] = e;
  } else {
    out[(long)b * D + d] = e;
  }
}

// ---------------------------------------------------------------- per-row int8 quantiser
// s = max(max|w|, 1e-8) / 127 (fp32);  q = clamp(rint(w / s), -127, 127);  s stored as bf16
// (round to nearest even) and optionally as the fp16 of that bf16 (app/convert_final.py:17-21,
// loader cast app/engine.py:241).
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ w,
                                                            int8_t* __restrict__ q,
                                                            uint16_t* __restrict__ s_bf16,
                                                            f16* __restrict__ s_f16, int K) {
  const long n = blockIdx.x;
  const float* wr = w + n * K;
  float mx = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(wr[k]));
  mx = wave_max(mx);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  const float amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
  int8_t* qr = q + n * K;
  for (int k = threadIdx.x; k < K; k += 256) {
    float v = rintf(wr[k] / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    qr[k] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) {
    const uint16_t sb = f32_to_bf16_rne(s);
    if (s_bf16) s_bf16[n] = sb;
    if (s_f16) s_f16[n] = (f16)__builtin_bit_cast(float, (uint32_t)sb << 16);
  }
}

// ---------------------------------------------------------------- RoPE table
// Llama-3 scaled frequencies (app/engine.py:28-43), same precision sequence:
//   e = fp32(2i) / fp32(hd);  p = fp32(base ** e);  f = fp32(1 / p)      (fp32 tensor ops)
//   band rule evaluated in double on f (Python floats), theta = fp32(result)
//   angle = fp32(fp32(pos) * theta);  table[pos, i] = (cos(angle), sin(angle)) as fp32
// pow, cos and sin are evaluated in double and rounded once to fp32.
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ out, int max_seq,
                                                         int hd, float base, double scale,
                                                         double low, double high, double old) {
  const int half = hd >> 1;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)max_seq * half) return;
  const int pidx = (int)(idx / half);
  const int i = (int)(idx - (long)pidx * half);
  const float e = (float)(2 * i) / (float)hd;
  const float pw = (float)pow((double)base, (double)e);
  const float f = 1.0f / pw;
  const double fd = (double)f;
  const double kPi = 3.141592653589793;
  const double wl = 2.0 * kPi / fd;
  const double lo_w = old / low, hi_w = old / high;
  double th;
  if (wl < hi_w) {
    th = fd;
  } else if (wl > lo_w) {
    th = fd / scale;
  } else {
    const double sm = (old / wl - low) / (high - low);
    th = (1.0 - sm) * fd / scale + sm * fd;
  }
  const float theta = (float)th;
  const float ang = (float)pidx * theta;
  out[idx * 2 + 0] = (float)cos((double)ang);
  out[idx * 2 + 1] = (float)sin((double)ang);
}

// Plain byte copy used to calibrate the HBM byte counters against a known traffic.
__global__ __launch_bounds__(256) void copy_bytes_kernel(const u32x4* __restrict__ src,
                                                         u32x4* __restrict__ dst, long n16) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n16; i += (long)gridDim.x * 256)
    dst[i] = __builtin_nontemporal_load(src + i);
}

}  // namespace ecd

using namespace ecd;

extern "C" {

int ecd_rmsnorm(const void* x, long ldx, const void* w, void* y, long ldy, int R, int D,
                float eps, void* stream) {
  if (!x || !w || !y || R <= 0 || D <= 0 || ldx < D || ldy < D) return ECD_EINVAL;
  const bool vec = (D % 512) == 0 && (ldx % 8) == 0 && (ldy % 8) == 0 &&
                   (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w) & 15) == 0;
  const dim3 g4((unsigned)((R + 3) / 4));
  hipStream_t st = (hipStream_t)stream;
  const f16 *xh = (const f16*)x, *wh = (const f16*)w;
  f16* yh = (f16*)y;
  switch (vec ? D / 512 : 0) {
    case 1: hipLaunchKernelGGL(rmsnorm_wave_kernel<1>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    case 2: hipLaunchKernelGGL(rmsnorm_wave_kernel<2>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    case 3: hipLaunchKernelGGL(rmsnorm_wave_kernel<3>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    case 4: hipLaunchKernelGGL(rmsnorm_wave_kernel<4>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    case 6: hipLaunchKernelGGL(rmsnorm_wave_kernel<6>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    case 8: hipLaunchKernelGGL(rmsnorm_wave_kernel<8>, g4, dim3(256), 0, st, xh, ldx, wh, yh, ldy, R, eps); break;
    default:
      hipLaunchKernelGGL(rmsnorm_kernel<256>, dim3(R), dim3(256), 0, st, xh, ldx, wh, yh, ldy, D, eps);
  }
  return ecd_launch_status();
}

int ecd_rope_kv_write(const void* qkv, const float* rope, const int64_t* pos, void* q, void* kc,
                      void* vc, int R, int S, int Hq, int Hk, int L, int HD, void* stream) {
  if (!qkv || !rope || !pos || !q || !kc || !vc || R <= 0 || S <= 0 || Hq <= 0 || Hk <= 0 ||
      L <= 0 || HD <= 0 || (HD & 1) || (Hq % Hk) != 0)
    return ECD_EINVAL;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(R), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)qkv, rope, pos, (f16*)q, (f16*)kc, (f16*)vc, S, Hq, Hk, L, HD);
  return ecd_launch_status();
}

int ecd_silu_mul(const void* x, void* y, int R, int F, void* stream) {
  if (!x || !y || R <= 0 || F <= 0) return ECD_EINVAL;
  dim3 grid((F + 2047) / 2048, R);
  hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const f16*)x,
                     (f16*)y, F);
  return ecd_launch_status();
}

int ecd_embed_sum_i8(const int64_t* tok, const void* table, const void* scales, long rows,
                     void* out, int B, int C, int D, int vocab, void* stream) {
  if (!tok || !table || !out || B <= 0 || C <= 0 || D <= 0 || vocab <= 0 || rows <= 0)
    return ECD_EINVAL;
  dim3 grid((D + 255) / 256, B);
  hipLaunchKernelGGL(embed_sum_kernel, grid, dim3(256), 0, (hipStream_t)stream, tok, table,
                     (const f16*)scales, (f16*)out, C, D, vocab, rows);
  return ecd_launch_status();
}

int ecd_embed_i8(const int64_t* tok, long tok_stride, const void* table, const void* scales,
                 long rows, int cb, int vocab, const void* even, void* out, int B, int D,
                 void* stream) {
  if (!tok || !table || !out || B <= 0 || D <= 0 || vocab <= 0 || cb < 0 || tok_stride <= 0 ||
      rows <= 0)
    return ECD_EINVAL;
  dim3 grid((D + 255) / 256, B);
  hipLaunchKernelGGL(embed_one_kernel, grid, dim3(256), 0, (hipStream_t)stream, tok, tok_stride,
                     table, (const f16*)scales, cb, vocab, rows, (const f16*)even, (f16*)out, D);
  return ecd_launch_status();
}

int ecd_quantize_rows_i8(const float* w, void* q, void* s_bf16, void* s_f16, int N, int K,
                         void* stream) {
  if (!w || !q || (!s_bf16 && !s_f16) || N <= 0 || K <= 0) return ECD_EINVAL;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(N), dim3(256), 0, (hipStream_t)stream, w,
                     (int8_t*)q, (uint16_t*)s_bf16, (f16*)s_f16, K);
  return ecd_launch_status();
}

int ecd_rope_table(float* out, int max_seq, int head_dim, double base, double scale, double low,
                   double high, double old, void* stream) {
  if (!out || max_seq <= 0 || head_dim <= 0 || (head_dim & 1) || !(high > low) || low <= 0)
    return ECD_EINVAL;
  const long n = (long)max_seq * (head_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, out, max_seq, head_dim, (float)base, scale, low, high,
                     old);
  return ecd_launch_status();
}

int ecd_copy_bytes(const void* src, void* dst, long nbytes, void* stream) {
  if (!src || !dst || nbytes <= 0 || (nbytes & 15) || ((uintptr_t)src & 15) ||
      ((uintptr_t)dst & 15))
    return ECD_EINVAL;
  const long n16 = nbytes / 16;
  long blocks = (n16 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)src, (u32x4*)dst, n16);
  return ecd_launch_status();
}

}  // extern "C"
