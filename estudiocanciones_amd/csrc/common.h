// Shared types and helpers for the gfx950 decode-path kernels.
//
// Every kernel in this library is launched on a caller-supplied hipStream_t,
// allocates nothing and never synchronises, so a whole frame of launches can be
// captured into one hipGraph by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ecdecode.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define ECD_WAVE 64

// Status codes (ECD_OK, ECD_EINVAL, ECD_ENOTSUP) come from ecdecode.h; positive values are
// hipError_t codes from a launch.

namespace ecd {

__device__ __forceinline__ float h2f(f16 h) { return (float)h; }
__device__ __forceinline__ f16 f2h(float f) { return (f16)f; }  // v_cvt_f16_f32: round to nearest even

// Four signed int8 codes packed in one dword -> two f16x2 holding the exact
// integer values.  u = q ^ 0x80 is q + 128 as an unsigned byte; placing it under
// the exponent byte 0x64 gives the half 1024 + u, and subtracting 1152 leaves q.
// Every step is exact (|q| <= 128 < 1024).
__device__ __forceinline__ void i8x4_to_f16(uint32_t v, f16x2& lo, f16x2& hi) {
  const uint32_t u = v ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0,u1
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2,u3
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = __builtin_bit_cast(f16x2, a) - bias;
  hi = __builtin_bit_cast(f16x2, b) - bias;
}

// 16 int8 codes (one 16-byte load) -> two f16x8 (codes 0..7 and 8..15).
__device__ __forceinline__ void i8x16_to_f16(const u32x4& v, f16x8& lo, f16x8& hi) {
  f16x2 a0, a1, b0, b1, c0, c1, d0, d1;
  i8x4_to_f16(v.x, a0, a1);
  i8x4_to_f16(v.y, b0, b1);
  i8x4_to_f16(v.z, c0, c1);
  i8x4_to_f16(v.w, d0, d1);
  lo = (f16x8){a0.x, a0.y, a1.x, a1.y, b0.x, b0.y, b1.x, b1.y};
  hi = (f16x8){c0.x, c0.y, c1.x, c1.y, d0.x, d0.y, d1.x, d1.y};
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Wave-wide scans and reductions on the VALU with DPP (no LDS crossbar round trips): row_shr
// 1, 2, 4, 8 inside each 16-lane row, then row_bcast:15 into rows 1 and 3 and row_bcast:31 into
// rows 2 and 3.  Lane l ends with the inclusive result over lanes 0..l; lanes whose DPP source
// is outside the row take `fill`, the operation's identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t fill) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)v, CTRL, ROWS, 0xF, false);
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x, uint32_t fill, Op op) {
  x = op(x, dpp_u32<0x111, 0xF>(x, fill));
  x = op(x, dpp_u32<0x112, 0xF>(x, fill));
  x = op(x, dpp_u32<0x114, 0xF>(x, fill));
  x = op(x, dpp_u32<0x118, 0xF>(x, fill));
  x = op(x, dpp_u32<0x142, 0xA>(x, fill));
  x = op(x, dpp_u32<0x143, 0xC>(x, fill));
  return x;
}
__device__ __forceinline__ uint32_t wave_incl_add_u32(uint32_t x) {
  return wave_incl_scan_u32(x, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
// reductions: the result in every lane (read from lane 63)
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = wave_incl_scan_u32(x, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = wave_incl_scan_u32(x, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
// fp32 sum in the scan's fixed order
__device__ __forceinline__ float wave_sum_dpp(float v) {
  const uint32_t r = wave_incl_scan_u32(
      __builtin_bit_cast(uint32_t, v), 0u, [](uint32_t a, uint32_t b) {
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
      });
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)r, 63));
}

// wait until at most N vector-memory operations of this wave are outstanding (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt at their maxima, i.e. not waited for)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_vm0() { wait_vm<0>(); }

// LDS DMA, one wave instruction: 16 bytes per lane from base + off (base wave-uniform, off a
// per-lane byte offset below 2^31) into LDS at dst + 16 * lane (dst uniform).  Issued from
// inline asm with M0 (the instruction's LDS base) saved and restored around it: with the
// compiler's builtin every later LDS read would wait for all outstanding DMA (vmcnt 0).
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, void* dst) {
  const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)dst;
  uint32_t keep;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(keep) : "v"(off), "s"(base), "s"(la) : "memory");
}

// RoPE on one interleaved pair with the rounding of eager fp16 ops: each product rounded to
// fp16, then the difference / sum in fp32 rounded to fp16; contraction off, so no product
// fuses into the sum (the codec estimator's apply_rope_vec).
__device__ __forceinline__ void rope_pair_f16(float x1, float x2, float co, float si, f16& o1,
                                              f16& o2) {
#pragma clang fp contract(off)
  o1 = (f16)((float)(f16)(x1 * co) - (float)(f16)(x2 * si));
  o2 = (f16)((float)(f16)(x1 * si) + (float)(f16)(x2 * co));
}

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __host__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Dense-numerics MFMA GEMM on a row-major [N, K] int8 weight (gemm_i8.hip); returns 1 without
// launching when the operands do not fit it.
int gemm_i8_rowmajor(const f16* x, long ldx, const int8_t* w, const f16* s, const f16* res,
                     long ldr, f16* y, long ldy, int M, int N, int K, hipStream_t st);

}  // namespace ecd

// Launch-error plumbing shared by the entry points.
static inline int ecd_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? ECD_OK : (int)e;
}
