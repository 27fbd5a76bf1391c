// Layer tail of a decode stack as one persistent launch per layer (gfx950).
//
// One launch computes, for a few rows (M <= 16), what the reference runs as five launches plus
// the next layer's first ones (app/engine.py:189-209; kernels app/kernels.py:11-180):
//
//   phase O    x1   = x + fp16(s_o * (W_o o))                      o-projection + residual
//   phase W13  mm   = fp16(silu(a)) * b,  a | b = fp16(s * (W1|W3 rms(x1, n2)))
//   phase W2   xout = x1 + fp16(s_2 * (W2 mm))                      down-projection + residual
//   phase QKV  q|k|v = fp16(s_q * (Wqkv rms(xout, n1'))), RoPE of q and k, q -> q_out,
//              k / v -> cache slot pos (the next layer's first step; skipped for the last layer)
//   phase ATT  the next layer's decode attention into o_next, q and the new K/V slots handed
//              over in tagged words (no gate)
//
// A head launch (HEAD) runs only phases QKV and ATT, on x = xin: a stack's layer 0.
//
// with the numerics of the per-op kernels (int8 codes x fp16 in fp32, fp16(acc * s), fp16
// residual add, the RMSNorm rounding points of app/kernels.py:58-67).
//
// Why one launch: at these row counts every GEMV is a weight stream of 2-50 MB, and a graph
// boundary between dependent launches costs ~3.5 us (dispatch gap, first-byte latency, store
// drain), more than the streaming time of the smaller matrices.  Here the grid is one
// workgroup per CU for the whole tail, and the phase boundaries are gates inside the kernel.
// A gate costs about as much as a launch boundary, but the weight stream does not stop at it:
// each compute wave holds its share of the next phase's weights in registers, loaded while
// the current phase computes and while the gate resolves, so HBM stays busy across phases.
//
// Workgroup: 8 compute waves + 1 loader wave.
//   * compute wave w owns K-chunks [w * C, (w + 1) * C) of every tile the workgroup has in a
//     phase (C = K / 512), keeps those weights in registers (packed lane-ordered 1 KB chunks,
//     int8 -> fp16 in registers, v_mfma_f32_16x16x32_f16 with the weights as A), reads the x
//     fragments from LDS and leaves its partial sums in LDS.  It never stores to global memory,
//     so waiting for its weights never waits for a store.
//   * after a gate has opened, each compute wave copies its own K-slice of the phase's
//     activation rows into LDS (global_load_lds); those copies queue behind the wave's weight
//     loads, which the phase needs next anyway.
//   * the loader wave polls the gates, adds up the eight partial sums in wave order, runs the
//     epilogue and stores the outputs.  Its queue holds only epilogue operands and stores, so
//     its wait for the stores before arriving at a gate never waits for a weight load.
// Tiles per workgroup (256 workgroups, 3B shapes): O 1 tile on 192 workgroups, W13 4 tiles,
// W2 1 tile (K = 8192) on 192 workgroups, QKV 1 or 2 tiles; the workgroups without an O or W2
// tile take the second QKV tiles, so every CU streams 336-416 KB per layer.
//
// Cross-workgroup visibility (CDNA3/4: one L2 per XCD, not coherent across XCDs).  Outputs
// read by other workgroups in the same launch (x1, mm, xout) are written with agent-scope
// relaxed atomic stores (global_store ... sc1: written through to memory); after its stores
// are acknowledged (s_waitcnt vmcnt(0)) the loader arrives at the gate with an atomic add on
// its group's counter (the 32 workgroups of blockIdx % 8, one XCD); the last of a group writes
// the group's done flag once for every group (each copy alone in its line), and each workgroup
// polls its group's eight copies with agent-scope loads.  No workgroup reads x1 / mm / xout before its gate has opened, and
// those lines are not in any L2 from earlier in the launch, so plain loads after the gate
// fetch them from memory.  The gate counters only ever grow, in step with the go value, so
// one 16 KB sync region serves every launch (each launch reads the go value at start).
// All workgroups are resident at once (grid = CU count, one workgroup per CU by LDS use);
// every wait on a gate is bounded, and a timeout sets *err and lets the kernel finish.
#pragma once
#include "attn_core.h"

#include <utility>

namespace ecd {
namespace tail {

constexpr int CW = 8;                // compute waves per workgroup
constexpr int NTHR = (CW + 1) * 64;  // plus the loader wave
constexpr int MR = 16;               // rows a launch takes (M <= MR; x tiles of R = 8 or 16 rows)
// LDS bytes per 64-column chunk of an x tile of R rows
__host__ __device__ constexpr int chb(int R) { return 128 * R; }
constexpr int ATT_SHORT = 128;       // caches of at most this many slots: one split per pair
constexpr int VSHORT = 8;            // caches of at most this many slots: the VALU attention
constexpr int VNEW = 2;              // ... written by at most this many rows per cache (S)
constexpr int ATT_KB_MAX = 16;       // workgroups per (row, kv head) pair, long caches

struct Args {
  const f16* o;    // [M, D] attention output of this layer
  const f16* xin;  // [M, D] layer input (residual of the O projection)
  const int8_t* wo;
  const f16* so;
  const f16* n2;
  const int8_t* w13;  // row-interleaved w1 | w3
  const f16* s13;
  const int8_t* w2;
  const f16* s2;
  // next layer's q|k|v step (wq == nullptr: last layer)
  const f16* n1;
  const int8_t* wq;
  const f16* sq;
  const float* rope;
  const int64_t* pos;
  f16* q;
  f16* kc;
  f16* vc;
  int S, Hq, Hk, L, HD;
  // outputs
  f16* x1;    // [M, D]
  f16* mm;    // [M, F]
  f16* xout;  // [M, D]
  // next layer's attention (ATT kernels): o_next [M, Hq * HD] from q and the caches
  f16* o_next;
  float scale;
  uint32_t* sync;  // 16 KB gate region, zero before the first launch
  uint32_t* err;   // made nonzero when a wait times out (bit 0 and the wait's ERR_ bit)
  float* ws;       // workspace, zero before the first launch on `sync`: split-W2 partial sums
                   // [D / 16][KS2][64][4] (KS2 > 1), the attention's per-workgroup partials
                   // [NB][G][2 + HD] (long caches) and the q|k|v hand-off [MR][Hq + 2 Hk][HD],
                   // all as tagged words
  int M, D, F;
  float eps;
  int spin_max;
  // a layer stack's last layer may end in a codebook head instead of the next layer's q|k|v:
  // y [M, yn] (row stride yld) = fp16(s_q * (Wq rms(xout, n1))), no attention (y == nullptr:
  // no head)
  f16* y;
  int yn, yld;
};

// One layer of a stack launch: its weights and buffers (the fields of Args that change from
// layer to layer; o and xin of layer l > 0 are o_next and xout of layer l - 1)
struct LayerRec {
  const int8_t* wo;
  const f16* so;
  const f16* n2;
  const int8_t* w13;
  const f16* s13;
  const int8_t* w2;
  const f16* s2;
  const f16* n1;
  const int8_t* wq;
  const f16* sq;
  f16* kc;
  f16* vc;
  f16* x1;
  f16* mm;
  f16* xout;
  f16* o_next;
  f16* y;  // the last layer only: the codebook head's output (wq, sq, n1 its weights and norm)
};

__device__ __forceinline__ void bar() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// LDS writes of this wave complete (vmcnt and expcnt not waited for)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

__device__ __forceinline__ void st_sc1_u64(f16* p, f16x4 v) {
  __hip_atomic_store((uint64_t*)p, __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1_u32(f16* p, f16x2 v) {
  __hip_atomic_store((uint32_t*)p, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1_f32x4(float* p, f32x4 v) {
  const u32x4 u = __builtin_bit_cast(u32x4, v);
  __hip_atomic_store((uint64_t*)p, (uint64_t)u.x | ((uint64_t)u.y << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store((uint64_t*)p + 1, (uint64_t)u.z | ((uint64_t)u.w << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 ld_sc1_f32x4(const float* p) {
  const uint64_t a = __hip_atomic_load((uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load((uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_bit_cast(f32x4, (u32x4){(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b,
                                           (uint32_t)(b >> 32)});
}
__device__ __forceinline__ uint32_t ld_sc1(const uint32_t* p) {
  return __hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Error word: bit 0 when any wait gave up, and one bit naming each wait that did.
constexpr uint32_t ERR_GATE_A = 2, ERR_GATE_B = 4, ERR_GATE_C = 8, ERR_SPLIT_W2 = 16,
                   ERR_HAND_VS = 32, ERR_HAND_Q = 64, ERR_NEW_SLOT = 128, ERR_MERGE = 256,
                   ERR_GATE_O = 512;
__device__ __forceinline__ void flag_err(uint32_t* err, uint32_t sites) {
  __hip_atomic_fetch_or(err, 1u | sites, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged words: 32 bits of data (one fp32, or two fp16) and the launch's epoch in one 8-byte
// word, stored and read whole at agent scope.  A reader that sees its epoch in a word sees that
// word's data of this launch, with no acknowledgement or flag between writer and reader.
__device__ __forceinline__ void put_tagged(uint64_t* p, uint32_t v, uint32_t epoch) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tagged(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t epoch) {
  return (uint32_t)(w >> 32) == epoch;
}

// Workspace float offsets: the attention partials after the split-W2 sums of a D-wide layer,
// the q|k|v hand-off after the partials of NB workgroups.
__device__ __forceinline__ long ws_att_offset(int D) { return (long)D * 128; }
__device__ __forceinline__ long ws_hand_offset(const Args& a, int NB) {
  return ws_att_offset(a.D) + (long)NB * (a.Hq / a.Hk) * (2 + a.HD) * 2;
}

// Pause between two looks of a poll: short while a wait is young (a gate resolves within a few
// microseconds), longer once it has lasted ~100 us, so that waiters of a late workgroup do not
// keep the lines its own stores and atomics go to busy with their reads.
__device__ __forceinline__ void poll_pause(int it) {
  if (it < 256)
    __builtin_amdgcn_s_sleep(1);
  else
    __builtin_amdgcn_s_sleep(32);
}

// Gate words (a 16 KB region): [64 (1 + g)] arrivals of group g's workgroups; flag word
// [GATE_FLAGS + 32 (8 x + g)] the done flag of group g as read by group x, one word alone in
// its 128-byte line, so that every line of the region has a single writer (the last arriver of
// one group) and each waiter polls eight lines of its own, with no second counter level between
// the last arrival and the flags.  The counters are never reset: every use of a gate adds
// exactly `per` to each group count and moves every flag by one, so the last arriver of a group
// is recognised from the go value the workgroup holds (all modulo 2^32; `per` divides 2^32).
// Called by one lane after this workgroup's output stores have been acknowledged.
constexpr int GATE_FLAGS = 1024;

__device__ __forceinline__ void gate_arrive(uint32_t* sync, int grp, uint32_t per, uint32_t go) {
  if (add_agent(sync + 64 * (1 + grp)) == (go + 1u) * per - 1u) {
#pragma unroll
    for (int x = 0; x < 8; ++x) store_agent(sync + GATE_FLAGS + 32 * (8 * x + grp), go + 1u);
  }
}

// The whole wave: lanes 0..7 poll group grp's view of the eight flags until each has reached
// go + 1 (a flag may already be one further: a group that passed this gate can complete the
// next one before a slow waiter looks).  Bounded by spin_max; the same result in every lane.
__device__ __forceinline__ bool gate_wait(const uint32_t* sync, int grp, uint32_t go,
                                          int spin_max, int lane) {
  const uint32_t* f = sync + GATE_FLAGS + 32 * (8 * grp + (lane & 7));
  for (int it = 0;; ++it) {
    const bool done = lane >= 8 || (int32_t)(ld_sc1(f) - (go + 1u)) >= 0;
    if (__builtin_amdgcn_ballot_w64(!done) == 0) return true;
    if (it >= spin_max) return false;
    poll_pause(it);
  }
}

// Activation copies into LDS are plain LDS DMA (L2-cacheable: the 32 workgroups of an XCD read
// the same rows, so all but the first hit its L2).  Every XCD's L2 starts a launch without the
// lines of this launch's activations, and none of x1 / mm / xout is read in a launch before
// the gate after which its writers' agent-scope stores are acknowledged, so the first read of
// a line fetches it from memory (the launch's inputs o and xin are final at its start).
// Activation rows [M, K] (row stride ld halfs) -> LDS x tile of R rows: chunk c (columns 64c ..
// 64c + 63) occupies chb(R) bytes as [grp 4][row R][16 halfs], grp = the 16-column group, i.e.
// exactly the B fragments of the two MFMAs of the chunk.  Each compute wave copies its own
// chunks [c0, c0 + C) to dst (the LDS address of chunk c0), R / 8 DMA instructions per chunk;
// in instruction i lane l moves 16 bytes: grp = i * 8 / R + l / 2R, row = (l >> 1) % R, half
// h = l & 1.  Rows past M repeat row M - 1 (their products land in output rows that are never
// stored).
template <int C, int R>
__device__ __forceinline__ void dma_rows(const f16* x, long ld, int M, int c0, unsigned char* dst,
                                         int lane) {
  constexpr int NI = R / 8;  // DMA instructions per chunk, 4 / NI column groups each
  const int row = (lane >> 1) % R, h = lane & 1, gl = lane / (2 * R);
  const int rs = row < M ? row : M - 1;
#pragma unroll
  for (int u = 0; u < C; ++u)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int grp = i * (4 / NI) + gl;
      lds_dma16(x, (uint32_t)(((long)rs * ld + 64 * (c0 + u) + 16 * grp + 8 * h) * 2),
                    dst + u * chb(R) + i * 1024);
      if (((u * NI + i) & 15) == 15) wait_vm<32>();  // at most ~48 DMA instructions in flight
    }
}

// The norm-weight columns of chunks [c0, c0 + C) -> LDS at the same offsets (C * 128 bytes:
// lanes past 8 C idle, so no lane reads past the vector)
template <int C>
__device__ __forceinline__ void dma_nw(const f16* v, int c0, unsigned char* dst, int lane) {
  static_assert(C * 8 <= 64, "one DMA instruction per wave");
  if (lane < C * 8) lds_dma16(v + 64 * c0, (uint32_t)(16 * lane), dst + 128 * c0);
}

// B fragments of chunk c of an R-row tile for this lane (row lane & 15; zero for rows >= R)
template <int R>
__device__ __forceinline__ void xfrag(const unsigned char* xs, int c, int lane, f16x8& fa,
                                      f16x8& fb) {
  const int row = lane & 15, grp = lane >> 4;
  if (row < R) {
    const unsigned char* p = xs + c * chb(R) + (grp * R + row) * 32;
    fa = *(const f16x8*)p;
    fb = *(const f16x8*)(p + 16);
  } else {
    fa = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    fb = fa;
  }
}

// RMSNorm of the fragments: fp16(fp16(x * inv) * nw)
__device__ __forceinline__ void rms_frag(f16x8& fa, f16x8& fb, const unsigned char* nws, int c,
                                         int lane, float inv) {
  const f16* nw = (const f16*)nws + 64 * c + 16 * (lane >> 4);
  const f16x8 na = *(const f16x8*)nw;
  const f16x8 nb = *(const f16x8*)(nw + 8);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    fa[e] = (f16)((float)fa[e] * inv) * na[e];
    fb[e] = (f16)((float)fb[e] * inv) * nb[e];
  }
}

// Sum of squares of this wave's chunks [c0, c0 + C) per row, reduced over the wave's four
// column groups; the per-wave sums go to ss[wave][row] in LDS.
template <int C, int R>
__device__ __forceinline__ void rms_partial(const unsigned char* xs, int c0, int lane, int wv,
                                            float* ss) {
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < C; ++u) {
    f16x8 fa, fb;
    xfrag<R>(xs, c0 + u, lane, fa, fb);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const f16x2 pa = (f16x2){fa[e], fa[e + 1]};
      const f16x2 pb = (f16x2){fb[e], fb[e + 1]};
      acc = __builtin_amdgcn_fdot2(pa, pa, acc, false);
      acc = __builtin_amdgcn_fdot2(pb, pb, acc, false);
    }
  }
  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 32, 64);
  if (lane < R) ss[wv * 16 + lane] = acc;
}

template <int R>
__device__ __forceinline__ float rms_inv(const float* ss, int lane, int K, float eps) {
  const int row = lane & 15;
  if (row >= R) return 0.f;
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < CW; ++w) t += ss[w * 16 + row];
  return 1.0f / sqrtf(t / (float)K + eps);
}

// 16 int8 codes -> two f16x8 holding q + 1152 exactly: the magic-number conversion of
// i8x16_to_f16 (q ^ 0x80 under the exponent byte 0x64 is the half 1024 + q + 128) without its
// final subtraction.  The GEMV then forms sum_k (q_k + 1152) x_k and removes 1152 sum_k x_k
// once per output.
__device__ __forceinline__ void i8x16_to_f16_biased(const u32x4& v, f16x8& lo, f16x8& hi) {
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = v[i] ^ 0x80808080u;
    h[2 * i] = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);      // bytes u0, u1
    h[2 * i + 1] = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2, u3
  }
  lo = __builtin_bit_cast(f16x8, (u32x4){h[0], h[1], h[2], h[3]});
  hi = __builtin_bit_cast(f16x8, (u32x4){h[4], h[5], h[6], h[7]});
}

// acc[t] += W_t x over chunks [c0, c0 + C) of this wave.  The weights enter the MFMAs as
// q + 1152 (two v_perm per four codes, no subtraction); the bias is removed at the end with
// 1152 sum_k x[m][k], formed by one extra MFMA per half-chunk whose A operand is the constant
// 1152 (its result is the same for every tile: lane l holds the sum of column l & 15).  Every
// product is exact in fp32; only the accumulation order of the fp32 sums differs from the
// unbiased form.
template <int NT, int C, int R>
__device__ __forceinline__ void mfma_chunks(f32x4 (&acc)[NT], const u32x4 (&w)[NT][C],
                                            const unsigned char* xs, const unsigned char* nws,
                                            int c0, int lane, float inv, bool rms) {
  const f16 kb = (f16)1152.0f;
  const f16x8 bias = (f16x8){kb, kb, kb, kb, kb, kb, kb, kb};
  f32x4 corr = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < C; ++u) {
    f16x8 fa, fb;
    xfrag<R>(xs, c0 + u, lane, fa, fb);
    if (rms) rms_frag(fa, fb, nws, c0 + u, lane, inv);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fa, corr, 0, 0, 0);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fb, corr, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f16x8 wa, wb;
      i8x16_to_f16_biased(w[t][u], wa, wb);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, fb, acc[t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] -= corr;
}

// acc[t] += W_t x over the weight chunks [U0, U0 + CN) of this wave (w[t][U0 ..]), whose x
// fragments sit at LDS chunks [c0, c0 + CN): mfma_chunks on part of the registers, no RMS.
template <int NT, int C, int R, int U0, int CN>
__device__ __forceinline__ void mfma_chunks_part(f32x4 (&acc)[NT], const u32x4 (&w)[NT][C],
                                                 const unsigned char* xs, int c0, int lane) {
  static_assert(U0 + CN <= C, "chunks within the registers");
  const f16 kb = (f16)1152.0f;
  const f16x8 bias = (f16x8){kb, kb, kb, kb, kb, kb, kb, kb};
  f32x4 corr = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < CN; ++u) {
    f16x8 fa, fb;
    xfrag<R>(xs, c0 + u, lane, fa, fb);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fa, corr, 0, 0, 0);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fb, corr, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f16x8 wa, wb;
      i8x16_to_f16_biased(w[t][U0 + u], wa, wb);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, fb, acc[t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] -= corr;
}

// Calls f(std::integral_constant<int, I>()) for I = 0 .. N - 1 (a loop with a constant index).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>());
}

// mfma_chunks with a hook after each chunk: after(integral_constant u) issues the next phase's
// weight loads into registers the finished chunks leave free, so the stream keeps going during
// the MFMAs.
template <int NT, int C, int R, typename After>
__device__ __forceinline__ void mfma_chunks_then(f32x4 (&acc)[NT], const u32x4 (&w)[NT][C],
                                                 const unsigned char* xs, const unsigned char* nws,
                                                 int c0, int lane, float inv, bool rms,
                                                 After after) {
  const f16 kb = (f16)1152.0f;
  const f16x8 bias = (f16x8){kb, kb, kb, kb, kb, kb, kb, kb};
  f32x4 corr = (f32x4){0.f, 0.f, 0.f, 0.f};
  static_for<C>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    f16x8 fa, fb;
    xfrag<R>(xs, c0 + u, lane, fa, fb);
    if (rms) rms_frag(fa, fb, nws, c0 + u, lane, inv);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fa, corr, 0, 0, 0);
    corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias, fb, corr, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f16x8 wa, wb;
      i8x16_to_f16_biased(w[t][u], wa, wb);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, fa, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, fb, acc[t], 0, 0, 0);
    }
    after(uc);
  });
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] -= corr;
}

template <bool NTL>
__device__ __forceinline__ u32x4 ldw(const int8_t* p) {
  if (NTL) return __builtin_nontemporal_load((const u32x4*)p);
  return *(const u32x4*)p;
}

template <int NT, int C, bool NTL>
__device__ __forceinline__ void load_w(u32x4 (&w)[NT][C], const int8_t* wp, const int (&tiles)[NT],
                                       int nch, int c0, int lane) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int u = 0; u < C; ++u)
      w[t][u] = ldw<NTL>(wp + ((long)tiles[t] * nch + c0 + u) * 1024 + 16 * lane);
}

// Chunks [u0, u1) of every tile, chunk-major.  LA > 0: paced -- before each load, wait until
// at most LA - 1 vector-memory operations of this wave are in flight.  A CU's outstanding reads
// queue in the memory system ahead of everything issued after them (the gate's atomics and
// polls, the activation copies, the epilogue stores), so the weight stream is kept at the depth
// HBM needs (LA KB per wave) instead of a whole phase ahead.
template <int NT, int C, bool NTL, int U0, int U1, int LA>
__device__ __forceinline__ void load_w_chunks(u32x4 (&w)[NT][C], const int8_t* wp,
                                              const int (&tiles)[NT], int nch, int c0, int lane) {
#pragma unroll
  for (int u = U0; u < U1; ++u)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (LA > 0) {
        wait_vm<(LA > 0 ? LA - 1 : 0)>();
        asm volatile("" ::: "memory");
      }
      w[t][u] = ldw<NTL>(wp + ((long)tiles[t] * nch + c0 + u) * 1024 + 16 * lane);
    }
}

template <int NT>
__device__ __forceinline__ void put_partials(unsigned char* ps, const f32x4 (&acc)[NT], int wv,
                                             int lane) {
#pragma unroll
  for (int t = 0; t < NT; ++t) *(f32x4*)(ps + ((wv * NT + t) * 64 + lane) * 16) = acc[t];
}

// sum of the eight waves' partials of tile t (wave order: the same sum in every launch); all
// eight LDS reads are issued before the first add
template <int NT>
__device__ __forceinline__ f32x4 sum_partials(const unsigned char* ps, int t, int lane) {
  f32x4 p[CW];
#pragma unroll
  for (int w = 0; w < CW; ++w) p[w] = *(const f32x4*)(ps + ((w * NT + t) * 64 + lane) * 16);
  f32x4 s = p[0];
#pragma unroll
  for (int w = 1; w < CW; ++w) s += p[w];
  return s;
}

__device__ __forceinline__ f16x4 scale4(const f32x4& acc, const f16x4& s) {
  f16x4 y;
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = (f16)(acc[r] * (float)s[r]);
  return y;
}

// ------------------------------------------------------------- next layer's attention phase
// Decode attention of app/kernels.py:111-167 for the M rows, their kv heads and the query heads
// of each (G = Hq / Hk), over cache slots [0, pos[r]], with the per-split core of the decode
// kernel (attn_core.h).  Short caches: one wave per (row, kv head) pair writes o directly.  Long
// caches: KB = NB / pairs workgroups per pair (att_pair gives a workgroup's pair p and part kq),
// split s = kq * 8 + wave of S = 8 KB splits (the split rule of app/kernels.py:120-127 with
// S splits); the loader merges its 8 waves' partials (log-sum-exp) into one per workgroup, and
// the pair's KB workgroups merge those and write o.  Same arithmetic as the split-combine
// kernel, summed in two levels.
// Long caches: pair p and part kq (of KB) of workgroup b.  Workgroups go to the XCDs round-robin
// (b % 8), so where each XCD's NB / 8 workgroups split into whole pairs, a pair's KB workgroups
// are taken from one XCD (their merge then stays within one L2); otherwise KB consecutive ids.
__device__ __forceinline__ void att_pair(int b, int NB, int KB, int& p, int& kq) {
  const int per = NB >> 3;
  if (per % KB == 0) {
    const int x = b & 7, i = b >> 3;
    p = x * (per / KB) + i / KB;
    kq = i % KB;
  } else {
    p = b / KB;
    kq = b - p * KB;
  }
}

// One wave's attention split; ring[0] holds its first K/V tile, read during the third gate.
template <int HD, int RING>
struct AttPre {
  KVTile<HD> ring[RING];
  long cbase;    // this pair's cache [L, HD] (K and V alike)
  int r, kh;     // row and kv head of the pair
  int lo, hi;    // the split's tokens held in the cache before the launch
  int p0;        // the cache's first slot written in this launch (L: none)
  int nlo, nhi;  // the split's tokens written in this launch, taken from the hand-off
  bool on;       // this wave runs a split
  bool staged;   // its third tile is copied into the wave's LDS slot (kv_stage)
};

// Split of this wave -- short caches: pair b + NB * wave, one split; long caches: pair and part
// kq of att_pair, split kq * 8 + wave of 8 KB -- and its first tile.  The S rows of a cache
// write consecutive slots p0 .. p0 + S - 1 (p0 = the position of its first row), and every slot
// below p0 is final before the launch: the split's cache part stops below p0, and its tokens
// from p0 on come from the hand-off, so no line of a slot written here is read.
template <int HD, int RING, bool KNT>
__device__ __forceinline__ void att_prefetch(const Args& a, int NB, int b, int wv, int lane,
                                             AttPre<HD, RING>& pf) {
  const int Hk = a.Hk, L = a.L;
  const int pairs = a.M * Hk;
  int p, ns, sp;
  if (L <= ATT_SHORT) {
    p = b + NB * wv;
    ns = 1;
    sp = 0;
  } else {
    const int KB = NB / pairs;
    int kq;
    att_pair(b, NB, KB, p, kq);
    ns = KB * CW;
    sp = kq * CW + wv;
  }
  pf.on = p < pairs;
  pf.staged = false;
  pf.lo = pf.hi = pf.nlo = pf.nhi = 0;
  if (!pf.on) return;
  pf.r = p / Hk;
  pf.kh = p - pf.r * Hk;
  const int c = pf.r / a.S;  // the row's cache
  pf.cbase = ((long)c * Hk + pf.kh) * (long)L * HD;
  split_range(a.pos, pf.r, L, ns, sp, pf.lo, pf.hi);
  const long praw = a.pos[c * a.S];
  pf.p0 = (praw >= 0 && praw < L) ? (int)praw : L;
  pf.nlo = max(pf.lo, pf.p0);
  pf.nhi = pf.hi;
  pf.hi = min(pf.hi, pf.p0);
  // Nontemporal slot loads (the slots are read once per step): they then stream without
  // displacing what the Infinity Cache holds for the frame's other launches.  Always with KNT
  // (the caller's choice: the depth decoder's weights stay resident), else for splits of more
  // than two tiles (caches of more than ~1000 slots); the two tiles of a short split load
  // faster as plain loads
  if (pf.lo < pf.hi) {
    if (KNT || pf.hi - pf.lo > 32)
      kv_load<HD, true>(pf.ring[0], a.kc + pf.cbase, a.vc + pf.cbase, pf.lo, pf.hi - 1, lane);
    else
      kv_load<HD, false>(pf.ring[0], a.kc + pf.cbase, a.vc + pf.cbase, pf.lo, pf.hi - 1, lane);
  }
}

// LDS slot (8 KB) of wave w's staged K/V tile: after the q|k|v phase's map (x tile, norm
// weights, row sums, the partials of two tiles) up to the W2 phase's x tile, then after the W2
// phase's partials.  Nothing else uses these bytes from the q|k|v phase to the attention's end.
template <int CD, int R, int CH>
__device__ __forceinline__ int stage_slot(int w) {
  constexpr int s0 = CD * CW * chb(R) + 2 * 64 * CD * CW + 512 + CW * 2 * 1024;
  constexpr int e0 = CH * CW * chb(R);
  constexpr int n0 = e0 > s0 ? (e0 - s0) / 8192 : 0;
  constexpr int s1 = e0 + CW * 1024;
  return w < n0 ? s0 + 8192 * w : s1 + 8192 * (w - n0);
}
template <int CD, int R, int CH>
constexpr int stage_end() {
  constexpr int s0 = CD * CW * chb(R) + 2 * 64 * CD * CW + 512 + CW * 2 * 1024;
  constexpr int e0 = CH * CW * chb(R);
  constexpr int n0 = e0 > s0 ? (e0 - s0) / 8192 : 0;
  return n0 >= CW ? s0 + 8192 * CW : e0 + CW * 1024 + 8192 * (CW - n0);
}

// One LDS DMA of 16 bytes per lane, nontemporal (lds_dma16 with the nt bit).
__device__ __forceinline__ void lds_dma16_nt(const void* base, uint32_t off, void* dst) {
  const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)dst;
  uint32_t keep;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "global_load_lds_dwordx4 %1, %2 nt\n\ts_mov_b32 m0, %0"
               : "=&s"(keep) : "v"(off), "s"(base), "s"(la) : "memory");
}

// A wave-uniform pointer in scalar registers (the LDS DMA takes its base there).  readfirstlane
// returns a signed int: each half goes through uint32_t before widening, or a low half with its
// top bit set would sign-extend over the high half.
__device__ __forceinline__ const f16* uniform_ptr(const f16* p) {
  const uint64_t u = (uint64_t)p;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  return (const f16*)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// The split's tile at t0 (tokens clamped to lim) into this wave's LDS slot dst, in kv_load's
// register order: DMA instruction j moves lane l's 16 bytes to dst + 1024 j + 16 l (the K
// fragments for j < 4, V rows j - 4 after them); kv_unstage (attn_core.h) reads them back.  The
// slots are read once per step: nontemporal.
__device__ __forceinline__ void kv_stage(const f16* kb, const f16* vb, int t0, int lim, int lane,
                                         unsigned char* dst) {
  constexpr int HD = 128;
  const int row = lane & 15, grp = lane >> 4;
  const f16* k0 = uniform_ptr(kb);
  const f16* v0 = uniform_ptr(vb);
  const uint32_t ko = (uint32_t)(((long)min(t0 + row, lim) * HD + 8 * grp) * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) lds_dma16_nt(k0, ko + 64 * i, dst + 1024 * i);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    lds_dma16_nt(v0, (uint32_t)(((long)min(t0 + 4 * grp + rr, lim) * HD + 8 * row) * 2),
                 dst + 1024 * (4 + rr));
}
// load_q from the hand-off words (row r's q at ((r * NQ + head * HD + d) / 2), two fp16 each),
// polled until every word this lane needs carries the epoch (bounded by spin_max).
template <int HD, int G>
__device__ __forceinline__ bool load_q_hand(f16x8 (&qf)[HD / 32], const uint64_t* hand, int r,
                                            int NQ, int kh, uint32_t ep, int lane, int spin_max) {
  const int row = lane & 15;
  const int grp = lane >> 4;
  const bool gv = row < G;
  const uint64_t* qp = hand + (((long)r * NQ + (long)(kh * G + (gv ? row : 0)) * HD + 8 * grp) >> 1);
  uint64_t w[HD / 32][4] = {};
  bool ok = true;
  for (int it = 0;; ++it) {
    bool ready = true;
    if (gv) {
#pragma unroll
      for (int i = 0; i < HD / 32; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          w[i][u] = get_tagged(qp + 16 * i + u);
          ready = ready && tag_is(w[i][u], ep);
        }
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
    if (it >= spin_max) {
      ok = false;
      break;
    }
    poll_pause(it);
  }
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
    qf[i] = __builtin_bit_cast(f16x8, (u32x4){(uint32_t)w[i][0], (uint32_t)w[i][1],
                                              (uint32_t)w[i][2], (uint32_t)w[i][3]});
  return ok;
}

// The split's last token, slot pn, as one more tile (token pn alone) from the hand-off: every
// lane holds one K word and one V word (HD / 2 words each; wk, wv as read with q, polled again
// until they carry the epoch, bounded by spin_max), then the lanes holding token 0 of the tile
// in the K and V registers gather their fp16 octets across lanes, and the tile updates the
// split state (the online softmax of attn_run_m, one more step).
template <int HD, int G>
__device__ __forceinline__ bool attn_new_slot(SplitStateM<HD, G>& ss, const f16x8 (&qf)[HD / 32],
                                              const uint64_t* hk, const uint64_t* hv, uint32_t ep,
                                              int pn, float scale, int lane, int spin_max,
                                              uint64_t wk, uint64_t wv) {
  static_assert(HD == 128, "one K word and one V word per lane");
  bool ok = true;
  for (int it = 0;; ++it) {
    if (__builtin_amdgcn_ballot_w64(!tag_is(wk, ep) || !tag_is(wv, ep)) == 0) break;
    if (it >= spin_max) {
      ok = false;
      break;
    }
    poll_pause(it);
    wk = get_tagged(hk + lane);
    wv = get_tagged(hv + lane);
  }
  const int k32 = (int)(uint32_t)wk, v32 = (int)(uint32_t)wv;
  const int row = lane & 15, grp = lane >> 4;
  KVTile<HD> t;
  // K: lane (0, grp) holds d = 8 grp + 32 c + e, i.e. words 4 grp + 16 c + e / 2
#pragma unroll
  for (int c = 0; c < KVTile<HD>::NKC; ++c) {
    u32x4 x;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      x[u] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * grp + 16 * c + u), k32);
    t.k[c] = row == 0 ? __builtin_bit_cast(f16x8, x) : (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  }
  // V: lane (row, 0) holds token 0 at rr = 0, d = 8 row + e, i.e. words 4 row + e / 2
  u32x4 y;
#pragma unroll
  for (int u = 0; u < 4; ++u) y[u] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * row + u), v32);
  t.v[0][0] = grp == 0 ? __builtin_bit_cast(f16x8, y) : (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int rr = 1; rr < 4; ++rr) t.v[rr][0] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  attn_tile_m<HD, G>(ss, ss.m_run, ss.l_run, qf, t, pn, pn + 1, scale, lane);
  return ok;
}

// Decode attention of app/kernels.py:111-167 for the M rows, their kv heads and the query heads
// of each (G = Hq / Hk), over cache slots [0, pos[r]], with the per-split core of the decode
// kernel (attn_core.h), on the splits att_prefetch assigned.  Short caches: the pair's one wave
// writes o directly.  Long caches: the loader merges its 8 waves' partials (log-sum-exp) into
// one per workgroup, and the pair's KB workgroups merge those (attention_merge).  Same
// arithmetic as the split-combine kernel, summed in two levels.  q and the new K/V slots come
// from the hand-off words of epoch `ep` (no gate after the q|k|v phase).
template <int HD, int G, int RING, bool KNT, bool WT>
__device__ __forceinline__ void attention_phase(const Args& a, unsigned char* smem, int wv,
                                                int lane, AttPre<HD, RING>& pf, uint32_t ep,
                                                const unsigned char* lt) {
  constexpr int PW = 2 + HD;  // floats per head of a partial: m, l, acc[HD]
  const int Hq = a.Hq;
  bar();  // X(ATT): the loader has read the q|k|v partials (LDS is free)
  if (!pf.on) {
    bar();  // P(ATT)
    return;
  }
  const f16* kb = a.kc + pf.cbase;
  const f16* vb = a.vc + pf.cbase;
  const int NQ = (Hq + 2 * a.Hk) * HD;
  const uint64_t* hw = (const uint64_t*)(a.ws + ws_hand_offset(a, gridDim.x));
  // splits of more than two tiles: the ring's other tiles go out before the q polls (the
  // polls then wait behind them in the CU's queue, which pays only when the stream is long),
  // as nontemporal loads (as in att_prefetch)
  const int ntiles = pf.hi > pf.lo ? (pf.hi - pf.lo + 15) / 16 : 0;
  const bool early = ntiles > 2;
  if (early) {
#pragma unroll
    for (int r = 1; r < RING; ++r)
      kv_load<HD, true>(pf.ring[r], kb, vb, pf.lo + 16 * r, pf.hi - 1, lane);
  }
  // the split's new slots: slot t from row (cache's first row + t - p0); the first one's K and
  // V words go out with the q polls (one round trip)
  auto hkv = [&](int t, const uint64_t*& hk, const uint64_t*& hv) {
    const long j = (long)(pf.r / a.S) * a.S + (t - pf.p0);
    hk = hw + ((j * NQ + (long)(Hq + pf.kh) * HD) >> 1);
    hv = hw + ((j * NQ + (long)(Hq + a.Hk + pf.kh) * HD) >> 1);
  };
  const uint64_t *hk = hw, *hv = hw;
  uint64_t nk = 0, nv = 0;
  if (pf.nlo < pf.nhi) {
    hkv(pf.nlo, hk, hv);
    nk = get_tagged(hk + lane);
    nv = get_tagged(hv + lane);
  }
  f16x8 qf[HD / 32];
  uint32_t bad = load_q_hand<HD, G>(qf, hw, pf.r, NQ, pf.kh, ep, lane, a.spin_max) ? 0u : ERR_HAND_Q;
  if (!early) {
#pragma unroll
    for (int r = 1; r < RING; ++r)
      if (r < ntiles) kv_load<HD, KNT>(pf.ring[r], kb, vb, pf.lo + 16 * r, pf.hi - 1, lane);
  }
  SplitStateM<HD, G> ss;
  attn_run_m<HD, G, RING, true, true, HD == 128 && RING == 2>(ss, qf, pf.ring, kb, vb, pf.lo,
                                                             pf.hi, a.scale, lane,
                                                             pf.staged ? lt : nullptr);
  for (int t = pf.nlo; t < pf.nhi; ++t) {
    if (t > pf.nlo) {
      hkv(t, hk, hv);
      nk = get_tagged(hk + lane);
      nv = get_tagged(hv + lane);
    }
    if (!attn_new_slot<HD, G>(ss, qf, hk, hv, ep, t, a.scale, lane, a.spin_max, nk, nv))
      bad |= ERR_NEW_SLOT;
  }
  if (bad && lane == 0) flag_err(a.err, bad);
  if (a.L <= ATT_SHORT) {
    attn_store_o_m<HD, G, WT>(ss, a.o_next + ((long)pf.r * Hq + pf.kh * G) * HD, lane);
    if constexpr (WT) wait_vm0();  // o acknowledged before the loader's next gate
    bar();  // P(ATT)
    return;
  }
  // this wave's partial -> LDS [wave][g][m, l, acc]
  attn_store_partial_m<HD, G>(ss, (float*)smem + wv * G * PW, PW, lane);
  wait_lgkm0();
  bar();  // P(ATT)
}

// Caches of at most VSHORT slots (the depth decoders'): the next layer's attention on the VALU,
// one wave per (row, kv head) pair, as the short-cache decode kernel computes it (no tiles, no
// MFMA): lane l owns dims [DPL l, DPL l + DPL) of every head (DPL = HD / 64, NW = DPL / 2
// words of two fp16).  Every cached slot below p0, the first slot this launch writes, is final
// before the launch: for head_dim 128 they are read before the third gate (16 registers); for
// wider heads, whose words would not fit beside the q|k|v weights, together with the first q
// polls.  q and the slots from p0 on come from the hand-off words.
template <int HD>
struct VPre {
  static constexpr int NW = HD / 128;
  static constexpr bool EARLY = NW == 1;  // cached words loaded before the third gate
  uint32_t k[VSHORT][NW], v[VSHORT][NW];
  long cbase;  // this lane's first word of the pair's cache [L, HD] (K and V alike)
  int last;    // the last cached slot below p0 (loads of later slots read it instead)
  int r, kh;   // row and kv head of the pair
  int p0;      // the cache's first slot written in this launch (L: none)
  int n;       // row r attends slots [0, n)
  bool on;     // this wave runs a pair
};

template <int HD>
__device__ __forceinline__ void vatt_load_cached(const Args& a, VPre<HD>& pf) {
#pragma unroll
  for (int t = 0; t < VSHORT; ++t) {
    const long off = pf.cbase + (long)min(t, pf.last) * HD;
#pragma unroll
    for (int w = 0; w < VPre<HD>::NW; ++w) {
      pf.k[t][w] = ((const uint32_t*)(a.kc + off))[w];
      pf.v[t][w] = ((const uint32_t*)(a.vc + off))[w];
    }
  }
}

template <int HD>
__device__ __forceinline__ void vatt_prefetch(const Args& a, int NB, int b, int wv, int lane,
                                              VPre<HD>& pf) {
  const int Hk = a.Hk, L = a.L;
  const int p = b + NB * wv;
  pf.on = p < a.M * Hk;
  pf.n = 0;
  pf.p0 = L;
  if (!pf.on) return;
  pf.r = p / Hk;
  pf.kh = p - pf.r * Hk;
  const int c = pf.r / a.S;  // the row's cache
  const long praw = a.pos[c * a.S];
  pf.p0 = (praw >= 0 && praw < L) ? (int)praw : L;
  const long pr = a.pos[pf.r];
  pf.n = (int)(pr + 1 < 0 ? 0 : (pr + 1 > L ? L : pr + 1));
  // slots past p0 are replaced by hand-off words: their loads read the last cached slot
  pf.last = max(min(pf.p0, L) - 1, 0);
  pf.cbase = ((long)c * Hk + pf.kh) * (long)L * HD + (HD / 64) * lane;
  if constexpr (VPre<HD>::EARLY) vatt_load_cached<HD>(a, pf);
}

// The pair's attention: q and the new slots polled from the hand-off words of epoch `ep`
// (bounded by spin_max), scores summed in fp32 over each lane's dims and across the wave, then
// the single-block softmax of app/kernels.py:111-153 (m = max, p = exp(s - m), l = sum of the
// unrounded p, acc = sum of fp16(p) v in fp32, o = fp16(acc / l)) into o_next.
template <int HD, int G, bool WT>
__device__ __forceinline__ void vattention_phase(const Args& a, int lane, VPre<HD>& pf,
                                                 uint32_t ep) {
  constexpr int NW = VPre<HD>::NW;
  constexpr int DPL = HD / 64;
  bar();  // X(ATT)
  if (!pf.on) {
    bar();  // P(ATT)
    return;
  }
  const int Hq = a.Hq, Hk = a.Hk;
  const long NQ = (long)(Hq + 2 * Hk) * HD;
  const uint64_t* hw = (const uint64_t*)(a.ws + ws_hand_offset(a, gridDim.x));
  const long c0 = (long)(pf.r / a.S) * a.S;  // the cache's first row
  if constexpr (!VPre<HD>::EARLY) vatt_load_cached<HD>(a, pf);  // in flight with the first polls
  uint32_t qw[G][NW], nk[VNEW][NW] = {}, nv[VNEW][NW] = {};
  bool ok = true;
  for (int it = 0;; ++it) {
    bool ready = true;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const uint64_t x =
            get_tagged(hw + ((pf.r * NQ + (long)(pf.kh * G + g) * HD) >> 1) + NW * lane + w);
        qw[g][w] = (uint32_t)x;
        ready = ready && tag_is(x, ep);
      }
#pragma unroll
    for (int i = 0; i < VNEW; ++i)
      if (pf.p0 + i < pf.n) {  // slot p0 + i from row c0 + i
        const long j = c0 + i;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const uint64_t xk = get_tagged(hw + ((j * NQ + (long)(Hq + pf.kh) * HD) >> 1) + NW * lane + w);
          const uint64_t xv =
              get_tagged(hw + ((j * NQ + (long)(Hq + Hk + pf.kh) * HD) >> 1) + NW * lane + w);
          nk[i][w] = (uint32_t)xk;
          nv[i][w] = (uint32_t)xv;
          ready = ready && tag_is(xk, ep) && tag_is(xv, ep);
        }
      }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
    if (it >= a.spin_max) {
      ok = false;
      break;
    }
    poll_pause(it);
  }
  if (!ok && lane == 0) flag_err(a.err, ERR_HAND_VS);
  // the new slots in place of the cached words read for them
#pragma unroll
  for (int t = 0; t < VSHORT; ++t)
#pragma unroll
    for (int i = 0; i < VNEW; ++i)
      if (t == pf.p0 + i)
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          pf.k[t][w] = nk[i][w];
          pf.v[t][w] = nv[i][w];
        }
  const int n = pf.n;
  float sc[G][VSHORT];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < VSHORT; ++t) {
      float d = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const f16x2 qa = __builtin_bit_cast(f16x2, qw[g][w]);
        const f16x2 ka = __builtin_bit_cast(f16x2, pf.k[t][w]);
        d += (float)qa.x * (float)ka.x;
        d += (float)qa.y * (float)ka.y;
      }
      sc[g][t] = d;
    }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < VSHORT; ++t) sc[g][t] = wave_sum_dpp(sc[g][t]);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < VSHORT; ++t) {
      sc[g][t] = t < n ? sc[g][t] * a.scale : -INFINITY;
      m = fmaxf(m, sc[g][t]);
    }
    float l = 0.f, acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
#pragma unroll
    for (int t = 0; t < VSHORT; ++t) {
      const float p = t < n ? __expf(sc[g][t] - m) : 0.f;
      l += p;
      const float ph = (float)(f16)p;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        // slots past n contribute nothing (their words may hold anything, even NaN)
        const f16x2 va = __builtin_bit_cast(f16x2, t < n ? pf.v[t][w] : 0u);
        acc[2 * w] += ph * (float)va.x;
        acc[2 * w + 1] += ph * (float)va.y;
      }
    }
    uint32_t* op = (uint32_t*)(a.o_next + ((long)pf.r * Hq + pf.kh * G + g) * HD + DPL * lane);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t ov =
          __builtin_bit_cast(uint32_t, (f16x2){(f16)(acc[2 * w] / l), (f16)(acc[2 * w + 1] / l)});
      if constexpr (WT)
        __hip_atomic_store(op + w, ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        op[w] = ov;
    }
  }
  if constexpr (WT) wait_vm0();  // o acknowledged before the loader's next gate
  bar();  // P(ATT)
}

// Log-sum-exp merge of n <= NMAX partials [i][g][m, l, acc[HD]] (stride `str` floats between
// partials) for head g and the columns d = lane + 64 k: the weights exp(m_i - max m) (0 for an
// empty part) and the sums in part order.  Every read is issued before the first use (one
// memory round trip).
template <int HD, int NMAX>
__device__ __forceinline__ void lse_merge(const float* src, int n, int str, int g, int lane,
                                          float& mo, float& lo, float (&ao)[(HD + 63) / 64],
                                          bool agent_scope) {
  constexpr int PW = 2 + HD;
  constexpr int NK = (HD + 63) / 64;
  auto rd = [&](const float* q) {
    return agent_scope ? __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)q,
                                                                     __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT))
                       : *q;
  };
  float m[NMAX], l[NMAX], v[NMAX][NK];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int k = 0; k < NK; ++k) v[i][k] = 0.f;
    if (i < n) {
      const float* q = src + i * str + g * PW;
      m[i] = rd(q);
      l[i] = rd(q + 1);
#pragma unroll
      for (int k = 0; k < NK; ++k)
        if (lane + 64 * k < HD) v[i][k] = rd(q + 2 + lane + 64 * k);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NMAX; ++i) mx = fmaxf(mx, m[i]);
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k) ao[k] = 0.f;
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    const float w = m[i] > -INFINITY ? __expf(m[i] - mx) : 0.f;
    ls += l[i] * w;
#pragma unroll
    for (int k = 0; k < NK; ++k) ao[k] += v[i][k] * w;
  }
  mo = mx;
  lo = ls;
}

// Long caches: the 8 waves' partials (LDS) -> this workgroup's partial [G][m, l, acc[HD]] in the
// workspace as 8-byte words (fp32 value, epoch), epoch = the gate count this launch reached
// after its last gate (the same in every workgroup, different in every launch on one sync
// region).  Then each of the pair's KB workgroups merges the KB partials for its HD / KB
// columns of every head as soon as all the words it needs carry the epoch (polls bounded by
// spin_max; lanes spread over parts x columns, G * HD / 64 value words and one (m, l) pair each,
// exchanged through LDS): the log-sum-exp sums of the per-op combine, parts in order, with no
// counter and no wait for this workgroup's own stores.  Returns false if a poll gave up.
template <int HD, int G, bool WT>
__device__ __forceinline__ bool attention_merge(const Args& a, unsigned char* smem, int NB, int b,
                                                int lane, uint32_t epoch) {
  static_assert(HD % 64 == 0, "value words spread evenly over the lanes");
  static_assert(G * ATT_KB_MAX <= 64, "one (m, l) pair per lane");
  constexpr int PW = 2 + HD;
  constexpr int NK = HD / 64;
  constexpr int NV = G * HD / 64;  // value words per lane
  const int pairs = a.M * a.Hk;
  if (a.L <= ATT_SHORT) return true;  // the waves wrote o
  const int KB = NB / pairs;
  int p, kq;
  att_pair(b, NB, KB, p, kq);
  const int r = p / a.Hk, kh = p - r * a.Hk;
  uint64_t* base = (uint64_t*)(a.ws + ws_att_offset(a.D)) + (long)p * KB * G * PW;
  uint64_t* part = base + (long)kq * G * PW;
  auto put = [&](uint64_t* q, float v) { put_tagged(q, __builtin_bit_cast(uint32_t, v), epoch); };
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mo, lo, ao[NK];
    lse_merge<HD, CW>((const float*)smem, CW, G * PW, g, lane, mo, lo, ao, false);
    if (lane == 0) {
      put(part + g * PW, mo);
      put(part + g * PW + 1, lo);
    }
#pragma unroll
    for (int k = 0; k < NK; ++k) put(part + g * PW + 2 + lane + 64 * k, ao[k]);
  }
  // word t = (part i, head g, column c) of this workgroup's columns d = kq * cw + c
  const int cw = HD / KB;  // KB divides HD
  const int gc = G * cw;
  const uint64_t* qv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int t = lane + 64 * j;
    const int i = t / gc, u = t - i * gc, g = u / cw;
    qv[j] = base + (long)i * G * PW + g * PW + 2 + kq * cw + (u - g * cw);
  }
  const bool hml = lane < KB * G;  // lane -> (part lane / G, head lane % G)
  const uint64_t* qm = base + (long)(lane / G) * G * PW + (lane % G) * PW;
  uint64_t wv[NV], wm = 0, wl = 0;
  bool ok = true;
  for (int it = 0;; ++it) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      wv[j] = get_tagged(qv[j]);
      ready = ready && tag_is(wv[j], epoch);
    }
    if (hml) {
      wm = get_tagged(qm);
      wl = get_tagged(qm + 1);
      ready = ready && tag_is(wm, epoch) && tag_is(wl, epoch);
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
    if (it >= a.spin_max) {
      ok = false;
      break;
    }
    poll_pause(it);
  }
  // exchange through LDS after the waves' partials (one wave: LDS accesses stay in order)
  float* sv = (float*)smem + CW * G * PW;  // [KB][G][cw]
  float* sml = sv + G * HD;                // [KB][G][m, l]
#pragma unroll
  for (int j = 0; j < NV; ++j) sv[lane + 64 * j] = __builtin_bit_cast(float, (uint32_t)wv[j]);
  if (hml) {
    sml[2 * lane] = __builtin_bit_cast(float, (uint32_t)wm);
    sml[2 * lane + 1] = __builtin_bit_cast(float, (uint32_t)wl);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  for (int u = lane; u < gc; u += 64) {
    const int g = u / cw;
    float mx = -INFINITY;
    for (int i = 0; i < KB; ++i) mx = fmaxf(mx, sml[2 * (i * G + g)]);
    float ls = 0.f, acc = 0.f;
    for (int i = 0; i < KB; ++i) {
      const float m = sml[2 * (i * G + g)];
      const float w = m > -INFINITY ? __expf(m - mx) : 0.f;
      ls += sml[2 * (i * G + g) + 1] * w;
      acc += sv[i * gc + u] * w;
    }
    f16* dst = a.o_next + ((long)r * a.Hq + kh * G + g) * HD + kq * cw + (u - g * cw);
    if constexpr (WT)
      __hip_atomic_store((uint16_t*)dst, __builtin_bit_cast(uint16_t, (f16)(acc / ls)),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      *dst = (f16)(acc / ls);
  }
  return ok;
}

// W2 phase rounds: a workgroup's K part of mm (C2 chunks per wave) is copied and multiplied in
// two rounds of half the chunks where the whole part would take more than 128 KB of LDS (16-row
// tiles of the 3072-wide layers: 256 KB)
__host__ __device__ constexpr int w2_rounds(int C2, int R) {
  return C2 * CW * chb(R) > 128 * 1024 ? 2 : 1;
}

// LDS map (bytes), per phase, for K = D columns: x tile [0, XD), norm weights [XD, XD + 2D),
// row sums [XD + 2D, + 512), partials after that; for the W2 phase (K = F): x tile [0, XF)
// (one round's chunks), partials [XF, XF + 8 KB).  A phase's partials never overlap its own x tile or norm weights
// (some waves still read those while others store partials); the next phase's x tile may
// overlap them (the loader has read the partials before it releases the next phase).
//
// Weight issue order of a compute wave (its vector-memory queue, in order): W_O and W13 at the
// start (and W2 where registers allow), then W2 and the next layer's q|k|v right after the W13
// MFMAs, so the weight stream does not wait for the gates.
//
// The lane index, opaque to the optimiser: in a stack launch the per-lane offsets derived from it
// are then computed inside each layer instead of being hoisted out of the layer loop and kept
// live (in registers the layer's weights need) across all of it.
__device__ __forceinline__ int lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
// The same for the wave index and the workgroup index (scalars), and what derives from them
__device__ __forceinline__ int wave_id() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return __builtin_amdgcn_readfirstlane(t >> 6);
}
__device__ __forceinline__ int block_id() {
  int b = blockIdx.x;
  asm volatile("" : "+v"(b));
  return __builtin_amdgcn_readfirstlane(b);
}

// One layer: tail_compute runs it on the compute waves, tail_loader on the loader wave (the two
// meet at the same barriers in the same order).  `go` (loader lane 0): the gate count this
// workgroup has reached; `bad`: the error bits of the loader's waits.  STK: a layer of a stack
// launch, whose attention output goes to memory by agent-scope stores; og: the layer's o is the
// previous layer's attention output from this launch, complete at the o gate (the weights go
// out before it).
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, bool HEAD, int R, bool VS,
          bool KNT, bool STK>
__device__ __forceinline__ void tail_compute(const Args& a, unsigned char* smem,
                                             const uint32_t& s_epoch, bool og, int wv) {
  constexpr int LA = 3;        // weight loads in flight per compute wave (paced issue)
  constexpr int C2 = CF / KS2;  // W2 chunks per compute wave (K split over KS2 workgroups)
  constexpr int W2H = w2_rounds(C2, R), CH = C2 / W2H;  // W2 rounds, chunks per round
  static_assert(C2 % W2H == 0, "whole chunks per round");
  const int lane = lane_id();
  const int NB = gridDim.x, b = block_id();
  const int D = a.D, F = a.F, M = a.M;
  const int nchD = CD * CW, nchF = CF * CW;  // D / 64, F / 64
  const bool has_next = a.wq != nullptr;
  // the next layer's attention runs in this launch (AHD > 0: its head_dim; AG query heads per
  // kv head), on q and the new K/V slots handed off in tagged words; caches
  // longer than ATT_SHORT slots are split over the KB workgroups of each (row, kv head) pair and
  // their 8 compute waves
  // YH: a 1024-wide decoder stack whose last layer may end in the codebook head (a.y set): its
  // q|k|v step is then the head GEMV on rms(xout, n1) into y, with no attention after it
  constexpr bool YH = STK && CD == 2 && VS;
  constexpr int NQ3 = YH ? 3 : 2;  // q|k|v (head) tiles a workgroup may take
  const bool yh = YH && a.y != nullptr;
  const bool att = AHD > 0 && has_next && !yh;

  // tiles of this workgroup (host: D / 16 <= NB, 2F / 16 == NT13 * NB, TQ <= 2 NB)
  const int TO = D >> 4;
  const int tO = b - (NB - TO);    // >= 0: one O tile
  // W2 (D / 16 tiles too): tile b (KS2 == 1), or tile b / KS2, K-part b % KS2 (host: D / 16 *
  // KS2 == NB), whose partial sums the K-part 0 workgroup adds up
  const int t2 = KS2 == 1 ? (b < TO ? b : -1) : b / KS2;
  const int ks2 = KS2 == 1 ? 0 : b % KS2;
  const int TQ = !has_next ? 0 : yh ? (a.yn + 15) >> 4 : ((a.Hq + 2 * a.Hk) * a.HD) >> 4;
  const int xtra = min(TQ, 2 * NB) - NB;
  // The two 16-column tiles whose hand-off words share a 128-byte line (tiles 2j, 2j + 1) go to
  // workgroups 8 apart, i.e. to one XCD: no line is written in pieces from two XCDs, which
  // agent-scope loads could read stale.  A permutation within each aligned block of 16.
  auto paired = [](int i) { return (i & ~15) + 2 * (i & 7) + ((i >> 3) & 1); };
  const int tq0 = b < TQ ? (b < (TQ & ~15) ? paired(b) : b) : -1;
  const int xb = b - (NB - xtra);  // this workgroup's index among those with a second tile
  const int tq1 = (xtra > 0 && xb >= 0) ? NB + (xb < (xtra & ~15) ? paired(xb) : xb) : -1;
  // a head's tiles past 2 NB (8197 columns: one) are the first workgroups' third tiles
  const int tq2 = YH && b < TQ - 2 * NB ? 2 * NB + b : -1;

  const int XD = nchD * chb(R);
  unsigned char* xs = smem;
  unsigned char* nws = smem + XD;
  float* ss = (float*)(smem + XD + 2 * D);
  unsigned char* psD = smem + XD + 2 * D + 512;  // partials of the K = D phases
  unsigned char* psF = smem + CH * CW * chb(R);  // partials of the W2 phase

  // ------------------------------------------------------------------ compute waves
  // attention splits: two K/V tiles in flight where the register budget allows it (G <= 3)
  constexpr int ARING = AG <= 3 ? 2 : 1;
  // tiled (MFMA) splits, or the VALU path for caches of at most VSHORT slots (VS)
  AttPre<(AHD > 0 && !VS ? AHD : 32), ARING> pf;
  VPre<(AHD > 0 && VS ? AHD : 128)> vpf;
  // long splits (more than two tiles) of the 8-row MFMA attention: the third tile goes into
  // an LDS slot of the wave during the q|k|v phase, so that it has arrived when q is seen
  constexpr bool STAGE = AHD == 128 && !VS && ARING == 2 && R == 8;
  unsigned char* lt = smem + stage_slot<CD, R, CH>(wv);
  auto stage = [&]() {
    if constexpr (STAGE) {
      if (att && pf.on && pf.hi - pf.lo > 32) {
        pf.staged = true;
        kv_stage(a.kc + pf.cbase, a.vc + pf.cbase, pf.lo + 32, pf.hi - 1, lane, lt);
      }
    }
  };
  const int c0D = wv * CD, c0F = ks2 * (C2 * CW) + wv * C2;
  u32x4 wq[NQ3][CD];
  int tq_t[NQ3];
  tq_t[0] = tq0 < 0 ? 0 : tq0;
  tq_t[1] = tq1 < 0 ? 0 : tq1;
  if constexpr (YH) tq_t[NQ3 - 1] = tq2 < 0 ? 0 : tq2;
  auto wq2 = [&]() -> u32x4(&)[2][CD] { return *(u32x4(*)[2][CD])wq; };
  auto tq2_t = [&]() -> const int(&)[2] { return *(const int(*)[2])tq_t; };
  if constexpr (!HEAD) {
    // this wave's slice of the attention output first (the inputs of this launch are final)
    if (!og) dma_rows<CD, R>(a.o, D, M, c0D, xs + c0D * chb(R), lane);
    u32x4 wo[1][CD];
    u32x4 w13[NT13][CD];
    const int to_t[1] = {tO < 0 ? 0 : tO};
    int t13[NT13];
#pragma unroll
    for (int t = 0; t < NT13; ++t) t13[t] = b * NT13 + t;
    if (tO >= 0) load_w<1, CD, NTL>(wo, a.wo, to_t, nchD, c0D, lane);
    load_w_chunks<NT13, CD, NTL, 0, 1, 0>(w13, a.w13, t13, nchD, c0D, lane);
    if (og) {
      bar();  // X(O): the previous layer's attention output is complete
      dma_rows<CD, R>(a.o, D, M, c0D, xs + c0D * chb(R), lane);
    }

    // phase O (x = o, already final: no gate).  Only waves with an O tile read the x tile; they
    // wait for this wave's o slice and W_O (the NT13 W13 loads issued after them may fly on)
    {
      f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
      if (tO >= 0) {
        if (og) wait_vm0();
        else wait_vm<NT13>();
        mfma_chunks<1, CD, R>(acc, wo, xs, nws, c0D, lane, 0.f, false);
      }
      put_partials<1>(psD, acc, wv, lane);
    }
    wait_lgkm0();
    bar();  // P(O)
    load_w_chunks<NT13, CD, NTL, 1, CD, LA>(w13, a.w13, t13, nchD, c0D, lane);
    u32x4 w2[1][C2];
    const int t2_t[1] = {t2 < 0 ? 0 : t2};

    // phase W13 (x = rms(x1, n2))
    bar();  // X(W13): x1 is complete
    dma_rows<CD, R>(a.x1, D, M, c0D, xs + c0D * chb(R), lane);
    dma_nw<CD>(a.n2, c0D, nws, lane);
    wait_vm0();
    rms_partial<CD, R>(xs, c0D, lane, wv, ss);
    wait_lgkm0();
    bar();  // S(W13)
    {
      const float inv = rms_inv<R>(ss, lane, D, a.eps);
      f32x4 acc[NT13];
#pragma unroll
      for (int t = 0; t < NT13; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
      // W2's chunks go out during the W13 MFMAs, into the registers each finished chunk frees
      mfma_chunks_then<NT13, CD, R>(acc, w13, xs, nws, c0D, lane, inv, true, [&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (t2 >= 0)
          load_w_chunks<1, C2, NTL, (u * C2) / CD, ((u + 1) * C2) / CD, LA>(w2, a.w2, t2_t, nchF,
                                                                            c0F, lane);
      });
      put_partials<NT13>(psD, acc, wv, lane);
    }
    wait_lgkm0();
    bar();  // P(W13)

    // the next layer's q|k|v weights go out during the second gate, into the registers the
    // W13 phase freed (HBM would idle there otherwise)
    if (YH && tq2 >= 0) load_w_chunks<NQ3, CD, NTL, 0, CD, LA>(wq, a.wq, tq_t, nchD, c0D, lane);
    else if (tq1 >= 0) load_w_chunks<2, CD, NTL, 0, CD, LA>(wq2(), a.wq, tq2_t(), nchD, c0D, lane);
    else if (tq0 >= 0)
      load_w_chunks<1, CD, NTL, 0, CD, LA>(*(u32x4(*)[1][CD])wq, a.wq, *(const int(*)[1])tq_t,
                                           nchD, c0D, lane);

    // phase W2 (x = mm)
    bar();  // X(W2): mm is complete
    if constexpr (W2H == 1) {
      // the workgroup's K part of mm: chunks c0F .. of F, at LDS chunks wv * C2 ..
      dma_rows<C2, R>(a.mm, F, M, c0F, xs + wv * C2 * chb(R), lane);
      wait_vm0();
      f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
      if (t2 >= 0) mfma_chunks<1, C2, R>(acc, w2, xs, nws, wv * C2, lane, 0.f, false);
      put_partials<1>(psF, acc, wv, lane);
    } else {
      // in rounds of CH chunks through this wave's LDS chunks wv * CH ..: a round's copy goes
      // out once the wave's LDS reads of the previous round are done (each wave reads only
      // its own chunks, so no barrier between rounds)
      f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
      static_for<W2H>([&](auto hc) {
        constexpr int h = decltype(hc)::value;
        if constexpr (h > 0) wait_lgkm0();
        dma_rows<CH, R>(a.mm, F, M, c0F + h * CH, xs + wv * CH * chb(R), lane);
        wait_vm0();
        if (t2 >= 0) mfma_chunks_part<1, C2, R, h * CH, CH>(acc, w2, xs, wv * CH, lane);
      });
      put_partials<1>(psF, acc, wv, lane);
    }
    wait_lgkm0();
    bar();  // P(W2)
  }

  if (has_next) {
    if constexpr (HEAD) {
      // head launch (x = xin, final at launch start): x slice, then the layer's q|k|v
      // weights, the only weights (all at once); the RMS waits for the x slice only
      dma_rows<CD, R>(a.xin, D, M, c0D, xs + c0D * chb(R), lane);
      dma_nw<CD>(a.n1, c0D, nws, lane);
      if (tq1 >= 0) {
        load_w_chunks<2, CD, NTL, 0, CD, 0>(wq2(), a.wq, tq2_t(), nchD, c0D, lane);
        wait_vm<2 * CD>();
      } else if (tq0 >= 0) {
        load_w_chunks<1, CD, NTL, 0, CD, 0>(*(u32x4(*)[1][CD])wq, a.wq, *(const int(*)[1])tq_t,
                                            nchD, c0D, lane);
        wait_vm<CD>();
      } else {
        wait_vm0();
      }
      rms_partial<CD, R>(xs, c0D, lane, wv, ss);
      if constexpr (AHD > 0 && VS) {
        if (att) vatt_prefetch<AHD>(a, NB, b, wv, lane, vpf);
      } else if constexpr (AHD > 0) {
        if (att) att_prefetch<AHD, ARING, KNT>(a, NB, b, wv, lane, pf);
        stage();
      }
      wait_lgkm0();
      bar();  // X(QKV)
    } else {
      // the next layer's first K/V tiles go out into the registers the W2 phase leaves free:
      // they stream during the third gate, and the loader's hand-off stores after the q|k|v
      // phase do not queue behind them
      if constexpr (AHD > 0 && VS) {
        if (att) vatt_prefetch<AHD>(a, NB, b, wv, lane, vpf);
      } else if constexpr (AHD > 0) {
        if (att) att_prefetch<AHD, ARING, KNT>(a, NB, b, wv, lane, pf);
      }
      // phase QKV (x = rms(xout, n1'))
      bar();  // X(QKV): xout is complete
      dma_rows<CD, R>(a.xout, D, M, c0D, xs + c0D * chb(R), lane);
      dma_nw<CD>(a.n1, c0D, nws, lane);
      wait_vm0();
      stage();
      rms_partial<CD, R>(xs, c0D, lane, wv, ss);
      wait_lgkm0();
    }
    bar();  // S(QKV)
    const float inv = rms_inv<R>(ss, lane, D, a.eps);
    f32x4 acc[NQ3];
#pragma unroll
    for (int t = 0; t < NQ3; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (YH && tq2 >= 0) mfma_chunks<NQ3, CD, R>(acc, wq, xs, nws, c0D, lane, inv, true);
    else if (tq1 >= 0)
      mfma_chunks<2, CD, R>(*(f32x4(*)[2])acc, wq2(), xs, nws, c0D, lane, inv, true);
    else if (tq0 >= 0)
      mfma_chunks<1, CD, R>(*(f32x4(*)[1])acc, *(u32x4(*)[1][CD])wq, xs, nws, c0D, lane, inv,
                            true);
    put_partials<NQ3>(psD, acc, wv, lane);
    wait_lgkm0();
    bar();  // P(QKV)
  }
  if constexpr (AHD > 0 && VS) {
    if (att) vattention_phase<AHD, AG, STK>(a, lane, vpf, s_epoch);
  } else if constexpr (AHD > 0) {
    if (att) attention_phase<AHD, AG, ARING, KNT, STK>(a, smem, wv, lane, pf, s_epoch, lt);
  }

}

template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, bool HEAD, int R, bool VS,
          bool KNT, bool STK>
__device__ __forceinline__ void tail_loader(const Args& a, unsigned char* smem, uint32_t& s_epoch,
                                            uint32_t& go, uint32_t& bad, bool og) {
  constexpr int LA = 3;        // weight loads in flight per compute wave (paced issue)
  constexpr int C2 = CF / KS2;  // W2 chunks per compute wave (K split over KS2 workgroups)
  constexpr int W2H = w2_rounds(C2, R), CH = C2 / W2H;  // W2 rounds, chunks per round
  static_assert(C2 % W2H == 0, "whole chunks per round");
  const int lane = lane_id();
  const int wv = wave_id();
  const int NB = gridDim.x, b = block_id();
  const int D = a.D, F = a.F, M = a.M;
  const int nchD = CD * CW, nchF = CF * CW;  // D / 64, F / 64
  const bool has_next = a.wq != nullptr;
  // the next layer's attention runs in this launch (AHD > 0: its head_dim; AG query heads per
  // kv head), on q and the new K/V slots handed off in tagged words; caches
  // longer than ATT_SHORT slots are split over the KB workgroups of each (row, kv head) pair and
  // their 8 compute waves
  // YH: a 1024-wide decoder stack whose last layer may end in the codebook head (a.y set): its
  // q|k|v step is then the head GEMV on rms(xout, n1) into y, with no attention after it
  constexpr bool YH = STK && CD == 2 && VS;
  constexpr int NQ3 = YH ? 3 : 2;  // q|k|v (head) tiles a workgroup may take
  const bool yh = YH && a.y != nullptr;
  const bool att = AHD > 0 && has_next && !yh;

  // tiles of this workgroup (host: D / 16 <= NB, 2F / 16 == NT13 * NB, TQ <= 2 NB)
  const int TO = D >> 4;
  const int tO = b - (NB - TO);    // >= 0: one O tile
  // W2 (D / 16 tiles too): tile b (KS2 == 1), or tile b / KS2, K-part b % KS2 (host: D / 16 *
  // KS2 == NB), whose partial sums the K-part 0 workgroup adds up
  const int t2 = KS2 == 1 ? (b < TO ? b : -1) : b / KS2;
  const int ks2 = KS2 == 1 ? 0 : b % KS2;
  const int TQ = !has_next ? 0 : yh ? (a.yn + 15) >> 4 : ((a.Hq + 2 * a.Hk) * a.HD) >> 4;
  const int xtra = min(TQ, 2 * NB) - NB;
  // The two 16-column tiles whose hand-off words share a 128-byte line (tiles 2j, 2j + 1) go to
  // workgroups 8 apart, i.e. to one XCD: no line is written in pieces from two XCDs, which
  // agent-scope loads could read stale.  A permutation within each aligned block of 16.
  auto paired = [](int i) { return (i & ~15) + 2 * (i & 7) + ((i >> 3) & 1); };
  const int tq0 = b < TQ ? (b < (TQ & ~15) ? paired(b) : b) : -1;
  const int xb = b - (NB - xtra);  // this workgroup's index among those with a second tile
  const int tq1 = (xtra > 0 && xb >= 0) ? NB + (xb < (xtra & ~15) ? paired(xb) : xb) : -1;
  // a head's tiles past 2 NB (8197 columns: one) are the first workgroups' third tiles
  const int tq2 = YH && b < TQ - 2 * NB ? 2 * NB + b : -1;

  const int XD = nchD * chb(R);
  unsigned char* xs = smem;
  unsigned char* nws = smem + XD;
  float* ss = (float*)(smem + XD + 2 * D);
  unsigned char* psD = smem + XD + 2 * D + 512;  // partials of the K = D phases
  unsigned char* psF = smem + CH * CW * chb(R);  // partials of the W2 phase

  // -------------------------------------------------------------------- loader wave
  const int me = lane & 15;        // output row of this lane's epilogue slot
  const int cg = 4 * (lane >> 4);  // its first column inside the tile
  const bool mrow = me < M;
  const int grp = b & 7;
  const uint32_t per = (uint32_t)(NB >> 3);
  if (og) {
    // the o gate: this workgroup's stores of the previous layer's attention output (the merge's,
    // and its compute waves', acknowledged before their last barrier) are acknowledged
    wait_vm0();
    if (lane == 0) gate_arrive(a.sync, grp, per, go);
  }

  // epilogue operands that do not depend on this launch's phases
  f16x4 so4 = {}, xr4 = {}, s2v = {};
  f16x4 s13v[NT13] = {};
  if constexpr (!HEAD) {
    if (tO >= 0) {
      so4 = *(const f16x4*)(a.so + 16 * tO + cg);
      if (mrow) xr4 = *(const f16x4*)(a.xin + (long)me * D + 16 * tO + cg);
    }
#pragma unroll
    for (int t = 0; t < NT13; ++t) s13v[t] = *(const f16x4*)(a.s13 + 16 * (b * NT13 + t) + cg);
    if (t2 >= 0) s2v = *(const f16x4*)(a.s2 + 16 * t2 + cg);
  }
  const int HD = a.HD, L = a.L;
  const int tq[3] = {tq0, tq1, tq2};
  f16x4 sqv[NQ3] = {};
  float cs[NQ3][4] = {};
  long p_raw = 0;
  if (has_next) {
    if (mrow) p_raw = a.pos[me];
    const long pc = p_raw < 0 ? 0 : (p_raw >= L ? L - 1 : p_raw);
#pragma unroll
    for (int i = 0; i < NQ3; ++i) {
      if (tq[i] < 0) continue;
      const int nb = 16 * tq[i] + cg;
      if (yh) {
        // the head's last tile reaches past its yn columns: clamped scale reads (the columns past
        // yn are not stored)
#pragma unroll
        for (int r = 0; r < 4; ++r) sqv[i][r] = a.sq[min(nb + r, a.yn - 1)];
        continue;
      }
      sqv[i] = *(const f16x4*)(a.sq + nb);
      const int h = nb / HD, d = nb - h * HD;
      if (h < a.Hq + a.Hk) {
        const float* c = a.rope + pc * HD + d;  // (cos, sin) of pairs d/2 and d/2 + 1
#pragma unroll
        for (int r = 0; r < 4; ++r) cs[i][r] = c[r];
      }
    }
  }

  if (og) {
    if (!gate_wait(a.sync, grp, __builtin_amdgcn_readfirstlane(go), a.spin_max, lane))
      bad |= ERR_GATE_O;
    ++go;
    bar();  // X(O)
  }

  if constexpr (!HEAD) {
    // phase O
    bar();  // P(O)
    if (tO >= 0) {
      const f16x4 y = scale4(sum_partials<1>(psD, 0, lane), so4);
      if (mrow) st_sc1_u64(a.x1 + (long)me * D + 16 * tO + cg, y + xr4);
    }
    wait_vm0();
    if (lane == 0) gate_arrive(a.sync, grp, per, go);
    if (!gate_wait(a.sync, grp, __builtin_amdgcn_readfirstlane(go), a.spin_max, lane))
      bad |= ERR_GATE_A;
    ++go;

    // phase W13 (the W2 epilogue's residual x1 is final now: read it before the weight stream of
    // the next phases is in flight)
    f16x4 r2 = {};
    if (t2 >= 0 && mrow)
      r2 = __builtin_bit_cast(f16x4, __hip_atomic_load((const uint64_t*)(a.x1 + (long)me * D + 16 * t2 + cg),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    bar();  // X(W13)
    bar();  // S(W13)
    bar();  // P(W13)
    {
      f16x2 o[NT13];
#pragma unroll
      for (int t = 0; t < NT13; ++t) {
        // interleaved w1 | w3 rows: (a_j, b_j, a_j+1, b_j+1), j = column / 2
        const f16x4 y = scale4(sum_partials<NT13>(psD, t, lane), s13v[t]);
        const float a0 = (float)y[0], a1 = (float)y[2];
        o[t].x = (f16)(a0 / (1.0f + expf(-a0))) * y[1];
        o[t].y = (f16)(a1 / (1.0f + expf(-a1))) * y[3];
      }
      if (mrow)
#pragma unroll
        for (int t = 0; t < NT13; ++t)
          st_sc1_u32(a.mm + (long)me * F + ((16 * (b * NT13 + t) + cg) >> 1), o[t]);
    }
    wait_vm0();
    if (lane == 0) gate_arrive(a.sync, grp, per, go);
    if (!gate_wait(a.sync, grp, __builtin_amdgcn_readfirstlane(go), a.spin_max, lane))
      bad |= ERR_GATE_B;
    ++go;

    // phase W2
    bar();  // X(W2)
    bar();  // P(W2)
    if (KS2 == 1) {
      if (t2 >= 0) {
        const f16x4 y = scale4(sum_partials<1>(psF, 0, lane), s2v) + r2;
        if (mrow) st_sc1_u64(a.xout + (long)me * D + 16 * t2 + cg, y);
      }
    } else {
      // K-parts 1 .. KS2 - 1 -> workspace as tagged words (epoch: the gate count after the
      // second gate, new in every launch), and on to the third gate without waiting for them;
      // the K-part 0 workgroup polls them, adds the KS2 parts in K order and stores xout
      uint64_t* wt = (uint64_t*)a.ws + ((long)t2 * KS2 * 64 + lane) * 4;
      const f32x4 part = sum_partials<1>(psF, 0, lane);
      const uint32_t ep2 = __builtin_amdgcn_readfirstlane(go);
      if (ks2 != 0) {
        // (a bit_cast of a vector element directly compiles to one element for every e)
        const float pe[4] = {part[0], part[1], part[2], part[3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) put_tagged(wt + ks2 * 256 + e, __builtin_bit_cast(uint32_t, pe[e]), ep2);
      } else {
        f32x4 acc = part;
#pragma unroll
        for (int k = 1; k < KS2; ++k) {
          uint64_t w[4];
          bool got = false;
          for (int it = 0;; ++it) {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = get_tagged(wt + k * 256 + e);
            got = tag_is(w[0], ep2) && tag_is(w[1], ep2) && tag_is(w[2], ep2) && tag_is(w[3], ep2);
            if (__builtin_amdgcn_ballot_w64(!got) == 0 || it >= a.spin_max) break;
            poll_pause(it);
          }
          if (__builtin_amdgcn_ballot_w64(!got) != 0) bad |= ERR_SPLIT_W2;
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] += __builtin_bit_cast(float, (uint32_t)w[e]);
        }
        const f16x4 y = scale4(acc, s2v) + r2;
        if (mrow) st_sc1_u64(a.xout + (long)me * D + 16 * t2 + cg, y);
      }
    }
  }

  if (has_next) {
    if constexpr (!HEAD) {
      // xout stores acknowledged (the split W2's K-parts 1 .. KS2 - 1 stored only tagged words,
      // which need no acknowledgement)
      if (KS2 == 1 || ks2 == 0) wait_vm0();
      if (lane == 0) gate_arrive(a.sync, grp, per, go);
      if (!gate_wait(a.sync, grp, __builtin_amdgcn_readfirstlane(go), a.spin_max, lane))
        bad |= ERR_GATE_C;
      ++go;
      if (lane == 0) s_epoch = go;
    } else {
      if (lane == 0) s_epoch = go + 1;
    }
    wait_lgkm0();
    bar();  // X(QKV)
    if constexpr (HEAD) {
      // the gate count moves on by one, arrivals only (every workgroup read it at launch
      // start), so that the next launch's epoch differs from this one's
      if (lane == 0) {
        gate_arrive(a.sync, grp, per, go);
        ++go;
      }
    }
    bar();  // S(QKV)
    bar();  // P(QKV)
    const bool pval = p_raw >= 0 && p_raw < L;
    // hand-off words of this launch's epoch: [row][q heads | k heads | v heads][HD] in pairs
    const uint32_t ep = __builtin_amdgcn_readfirstlane(go);
    const int NQ = (a.Hq + 2 * a.Hk) * HD;
    uint64_t* hw = (uint64_t*)(a.ws + ws_hand_offset(a, NB));
#pragma unroll
    for (int i = 0; i < NQ3; ++i) {
      if (tq[i] < 0) continue;
      const f16x4 y = scale4(sum_partials<NQ3>(psD, i, lane), sqv[i]);
      if (!mrow) continue;
      if (yh) {  // the codebook head: logits of row me, columns nb .. nb + 3 (those below yn)
        const int nb = 16 * tq[i] + cg;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < a.yn) a.y[(long)me * a.yld + nb + r] = y[r];
        continue;
      }
      const int nb = 16 * tq[i] + cg;
      const int h = nb / HD, d = nb - h * HD;
      f16x4 o;
      if (h < a.Hq + a.Hk) {
        const float x0 = (float)y[0], x1 = (float)y[1], x2 = (float)y[2], x3 = (float)y[3];
        o[0] = (f16)(x0 * cs[i][0] - x1 * cs[i][1]);
        o[1] = (f16)(x1 * cs[i][0] + x0 * cs[i][1]);
        o[2] = (f16)(x2 * cs[i][2] - x3 * cs[i][3]);
        o[3] = (f16)(x3 * cs[i][2] + x2 * cs[i][3]);
      } else {
        o = y;
      }
      f16* dst = nullptr;
      if (h < a.Hq) {
        dst = a.q + ((long)me * a.Hq + h) * HD + d;
      } else if (pval) {
        const int bb = me / a.S;
        const int kh = h < a.Hq + a.Hk ? h - a.Hq : h - a.Hq - a.Hk;
        dst = (h < a.Hq + a.Hk ? a.kc : a.vc) + (((long)bb * a.Hk + kh) * L + p_raw) * HD + d;
      }
      if (att) {  // this launch's attention reads the hand-off words, not q or the caches
        const uint64_t ov = __builtin_bit_cast(uint64_t, o);
        uint64_t* hp = hw + (((long)me * NQ + nb) >> 1);
        put_tagged(hp, (uint32_t)ov, ep);
        put_tagged(hp + 1, (uint32_t)(ov >> 32), ep);
      }
      if (dst) *(f16x4*)dst = o;
    }
    if constexpr (AHD > 0) {
      if (!att) return;
      bar();  // X(ATT)
      bar();  // P(ATT)
      if constexpr (!VS)
        if (!attention_merge<AHD, AG, STK>(a, smem, NB, b, lane, __builtin_amdgcn_readfirstlane(go)))
          bad |= ERR_MERGE;
    }
  }
}

// One launch per layer tail (a head launch: HEAD).
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, bool HEAD, int R, bool VS,
          bool KNT>
__global__ __launch_bounds__(NTHR) void layer_tail_kernel(const Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ uint32_t s_epoch;  // this launch's epoch (loader -> compute waves)
  if (threadIdx.x < CW * 64) {
    tail_compute<CD, CF, NT13, KS2, AHD, AG, NTL, HEAD, R, VS, KNT, false>(
        a, smem, s_epoch, false, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    return;
  }
  const bool ld0 = threadIdx.x == CW * 64;  // the loader's lane 0
  uint32_t go = 0, bad = 0;
  if (ld0) go = ld_sc1(a.sync + GATE_FLAGS + 32 * 8 * (blockIdx.x & 7));  // (all flags equal here)
  tail_loader<CD, CF, NT13, KS2, AHD, AG, NTL, HEAD, R, VS, KNT, false>(a, smem, s_epoch, go, bad,
                                                                         false);
  if (ld0 && bad) flag_err(a.err, bad);
}

// Layer l of a stack: the shared fields of a0 with the record's pointers (o and xin of l > 0 from
// layer l - 1's record).  The records are read through the constant address space: they do not
// change during the launch, scalar loads fetch them, and the compiler takes the pointers read
// from there to be global memory (global, not flat, instructions).
typedef const __attribute__((address_space(4))) LayerRec CLayerRec;
typedef const __attribute__((address_space(4))) Args CArgs;
__device__ __forceinline__ Args stack_args(const LayerRec* plan, int l) {
  CLayerRec* c = (CLayerRec*)plan;
  // the shared fields are read from the kernel arguments again for every layer (an opaque
  // pointer to them), not held in scalar registers across the layer loop
  Args a;
#if __HIP_DEVICE_COMPILE__  // (the host pass only parses this function)
  CArgs* ap = (CArgs*)__builtin_amdgcn_kernarg_segment_ptr();  // a0: the first argument
  asm volatile("" : "+s"(ap));
  __builtin_memcpy(&a, ap, sizeof(Args));
#endif
  a.wo = c[l].wo; a.so = c[l].so; a.n2 = c[l].n2; a.w13 = c[l].w13; a.s13 = c[l].s13;
  a.w2 = c[l].w2; a.s2 = c[l].s2; a.n1 = c[l].n1; a.wq = c[l].wq; a.sq = c[l].sq;
  a.kc = c[l].kc; a.vc = c[l].vc; a.x1 = c[l].x1; a.mm = c[l].mm; a.xout = c[l].xout;
  a.o_next = c[l].o_next;
  a.y = c[l].y;
  if (l > 0 || a.o == nullptr) {  // (l = 0 without o: a later part of a longer plan)
    a.o = c[l - 1].o_next;
    a.xin = c[l - 1].xout;
  }
  return a;
}

// A stack of layer tails in one launch: layer l's attention output (its o_next) is layer l + 1's
// o, and its output xout is layer l + 1's input.  Between two layers the workgroups meet at one
// more gate (o complete) instead of a launch boundary, and the next layer's O and first W13
// weights stream while they wait.  Every activation buffer of a stack is its layer's own, so no
// XCD's L2 holds a line of one before its writers have finished it.
// NLU > 0: exactly NLU layers, unrolled (straight-line code: no layer loop whose
// loop-invariant values would be held in registers across it); nl is then NLU.
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, int R, bool VS, bool KNT,
          int NLU = 0>
__global__ __launch_bounds__(NTHR) void layer_stack_kernel(const Args a0,
                                                           const LayerRec* __restrict__ plan,
                                                           int nl) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ uint32_t s_epoch;
  if (threadIdx.x < CW * 64) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    auto layer = [&](int l) __attribute__((always_inline)) {
      tail_compute<CD, CF, NT13, KS2, AHD, AG, NTL, false, R, VS, KNT, true>(
          stack_args(plan, l), smem, s_epoch, l > 0, wv);
    };
    if constexpr (NLU > 0)
      static_for<NLU>([&](auto lc) { layer(decltype(lc)::value); });
    else
      for (int l = 0; l < nl; ++l) layer(l);
    return;
  }
  const bool ld0 = threadIdx.x == CW * 64;
  uint32_t go = 0, bad = 0;
  if (ld0) go = ld_sc1(a0.sync + GATE_FLAGS + 32 * 8 * (blockIdx.x & 7));
  auto layer = [&](int l) __attribute__((always_inline)) {
    tail_loader<CD, CF, NT13, KS2, AHD, AG, NTL, false, R, VS, KNT, true>(
        stack_args(plan, l), smem, s_epoch, go, bad, l > 0);
  };
  if constexpr (NLU > 0)
    static_for<NLU>([&](auto lc) { layer(decltype(lc)::value); });
  else
    for (int l = 0; l < nl; ++l) layer(l);
  if (ld0 && bad) flag_err(a0.err, bad);
}

inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev]) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
    cus[dev] = p.multiProcessorCount;
  }
  return cus[dev];
}

// Dynamic LDS bytes of a launch: the phases' x tiles, norm weights, row sums and partials, the
// attention's partials and merge exchange, the staged K/V tiles of long splits
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, int R, bool VS>
int tail_lds(int D) {
  const int xd = CD * CW * chb(R), xf = CF / KS2 / w2_rounds(CF / KS2, R) * CW * chb(R);
  const int ldsD = xd + 2 * D + 512 + CW * (NT13 > 2 ? NT13 : 2) * 1024;
  const int ldsF = xf + CW * 1024;
  // attention: the waves' partials, then the merge's exchange
  const int ldsA = AHD > 0 && !VS ? (CW * AG * (2 + AHD) + AG * AHD + 2 * ATT_KB_MAX * AG) * 4 : 0;
  int lds = ldsD > ldsF ? ldsD : ldsF;
  if (lds < ldsA) lds = ldsA;
  // the staged K/V tiles of long attention splits (8-row MFMA attention)
  constexpr int C2 = CF / KS2, CH = C2 / w2_rounds(C2, R);
  constexpr int lde = AHD == 128 && !VS && AG <= 3 && R == 8 ? stage_end<CD, R, CH>() : 0;
  if (lds < lde) lds = lde;
  return lds;
}

// dynamic LDS beyond the default limit (the kernel's static LDS comes on top of it), raised once
// per kernel to the largest size launched
inline int raise_lds(const void* fn, int lds, int& attr) {
  if (lds > attr) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return (int)e;
    attr = lds;
  }
  return 0;
}

template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, bool HEAD, int R, bool VS,
          bool KNT = false>
int launch(const Args& a, int nb, hipStream_t st) {
  const int lds = tail_lds<CD, CF, NT13, KS2, AHD, AG, R, VS>(a.D);
  static int attr = 0;
  const auto fn = layer_tail_kernel<CD, CF, NT13, KS2, AHD, AG, NTL, HEAD, R, VS, KNT>;
  if (const int rc = raise_lds((const void*)fn, lds, attr)) return rc;
  hipLaunchKernelGGL(fn, dim3(nb), dim3(NTHR), lds, st, a);
  return ecd_launch_status();
}

// A stack instantiation runs only if its code needs no scratch memory: the dispatcher may hold
// back waves whose scratch is not yet available, and a persistent launch must have every
// workgroup resident (register spills would also break its pipelined weight stream).  Cached.
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, int R, bool VS, bool KNT,
          int NLU = 0>
bool stack_scratch_free() {
  static int ok = -1;
  if (ok < 0) {
    hipFuncAttributes fa;
    const auto fn = layer_stack_kernel<CD, CF, NT13, KS2, AHD, AG, NTL, R, VS, KNT, NLU>;
    ok = hipFuncGetAttributes(&fa, (const void*)fn) == hipSuccess && fa.localSizeBytes == 0;
  }
  return ok;
}

// NLU > 0: the nl layers as nl / NLU launches of NLU layers each (the parts after the first
// take their o and xin from the record before them: Args o == nullptr).
template <int CD, int CF, int NT13, int KS2, int AHD, int AG, bool NTL, int R, bool VS, bool KNT,
          int NLU = 0>
int launch_stack(const Args& a, const LayerRec* plan, int nl, int nb, hipStream_t st) {
  if (NLU > 0 && nl % NLU) return ECD_ENOTSUP;
  if (!stack_scratch_free<CD, CF, NT13, KS2, AHD, AG, NTL, R, VS, KNT, NLU>()) return ECD_ENOTSUP;
  const int lds = tail_lds<CD, CF, NT13, KS2, AHD, AG, R, VS>(a.D);
  static int attr = 0;
  const auto fn = layer_stack_kernel<CD, CF, NT13, KS2, AHD, AG, NTL, R, VS, KNT, NLU>;
  if (const int rc = raise_lds((const void*)fn, lds, attr)) return rc;
  if constexpr (NLU == 0) {
    hipLaunchKernelGGL(fn, dim3(nb), dim3(NTHR), lds, st, a, plan, nl);
    return ecd_launch_status();
  } else {
    Args ak = a;
    for (int k = 0; k < nl; k += NLU) {
      if (k > 0) ak.o = ak.xin = nullptr;
      hipLaunchKernelGGL(fn, dim3(nb), dim3(NTHR), lds, st, ak, plan + k, NLU);
      if (const int rc = ecd_launch_status()) return rc;
    }
    return 0;
  }
}

}  // namespace tail
}  // namespace ecd

namespace ecd {

// Attention in the launch: (head_dim, query heads per kv head) instantiated, and the work split
// fits the grid (long caches: NB / pairs workgroups per (row, kv head) pair).
static inline bool tail_att_ok(int nb, int M, int D, int Hq, int Hk, int HD, int L) {
  if (Hk <= 0 || Hq % Hk) return false;
  const int G = Hq / Hk, pairs = M * Hk;
  // head_dim 128 with 3 or 4 query heads per kv head at any length; head_dim 384 with 2 (the
  // reference's depth decoder) on caches of at most VSHORT slots (the VALU path)
  if (!(HD == 128 && (G == 3 || G == 4)) && !(HD == 384 && G == 2 && L <= tail::VSHORT))
    return false;
  // 3072-wide layers take more than 8 rows only as the reference decoder's first pass
  if (D == 3072 && M > 8 && !(HD == 384 && G == 2 && L <= tail::VSHORT)) return false;
  if (L <= tail::ATT_SHORT) return pairs <= nb * tail::CW;
  // KB = nb / pairs workgroups per pair, each merging HD / KB columns
  const int kb = nb / pairs;
  return nb % pairs == 0 && kb <= tail::ATT_KB_MAX && HD % kb == 0;
}
}  // namespace ecd
