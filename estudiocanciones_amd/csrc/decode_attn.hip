// GQA flash-decoding attention over the static KV cache, gfx950.
//
// Reference semantics (app/kernels.py:111-167): row r (batch b = r / S) attends to cache
// slots [0, pos[r]] of kv head kh with its G = Hq / Hk query heads; scores are
// fp32( q . k ) * scale, softmax with natural exp and a running max, the probabilities
// are rounded to fp16 before the P.V product (fp32 accumulation), the running sum uses
// the unrounded fp32 probabilities.  The attended range is cut into `nsplit` chunks of
// ceil(ceil(len / nsplit) / 16) * 16 tokens; each split writes (m, l, acc) partials that
// the combine kernel merges with a log-sum-exp rescale (empty splits have m = -inf).
//
// Kernel shape: one wave per (split, kv head, row).  Each 16-token tile is
//   S^T = K_tile . Q^T   on v_mfma_f32_16x16x32_f16: the K rows are the A operand (lane l
//                        loads 16 contiguous bytes of token t0 + (l & 15)), Q^T the B operand
//                        (query head g = l & 15, zero for g >= G), so lane l ends holding
//                        scores of tokens t0 + 4 (l >> 4) + r, r = 0..3, for head l & 15;
//   O^T += V^T . P       on v_mfma_f32_16x16x16_f16: the scores' lane layout is the B operand
//                        as it stands, and lane l's V rows (d-chunk 8 (l & 15) .. +8 of tokens
//                        t0 + 4 (l >> 4) + r) are the A operand of V^T for the output rows
//                        d = 8 m + b, one MFMA per b (plus 128-wide repeats): no lane exchange,
//                        the tile's 16 tokens are summed inside the MFMA.
// Each K and V byte of the attended range is read once per (row, kv head): the G query
// heads of a group share it (no repeat_kv copy).
#include <mutex>

#include "attn_core.h"

namespace ecd {

// Tiles in flight per wave: four for head_dim <= 128, two for 256, one for wider heads.
constexpr int attn_ring(int HD) { return HD <= 128 ? 4 : (HD <= 256 ? 2 : 1); }

template <int HD, int G>
__global__ __launch_bounds__(64) void decode_attn_kernel(
    const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
    const int64_t* __restrict__ pos, f16* __restrict__ o, float* __restrict__ pm,
    float* __restrict__ pl, float* __restrict__ pa, int S, int Hq, int Hk, int L, float scale,
    int nsplit) {
  static_assert(HD % 32 == 0 && HD <= 512, "head_dim must be a multiple of 32");
  static_assert(G >= 1 && G <= 16, "query heads per kv head must be 1..16");
  constexpr int NDP = SplitStateM<HD, G>::NDP;
  const int lane = threadIdx.x;
  const int n = lane & 15;  // query head of this lane's outputs
  const int grp = lane >> 4;
  const int sp = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
  const int b = r / S;
  const long cbase = ((long)b * Hk + kh) * (long)L * HD;
  // one split starts at slot 0: its first tile is loaded before the attended length is known
  // (rows clamped to the cache, masked later), so the position read and the tile overlap
  KVTile<HD> ring[attn_ring(HD)];
  if (nsplit == 1) kv_load<HD>(ring[0], kc + cbase, vc + cbase, 0, L - 1, lane);
  f16x8 qf[HD / 32];
  load_q<HD, G>(qf, q, r, Hq, kh, lane);
  int lo, hi;
  split_range(pos, r, L, nsplit, sp, lo, hi);
  if (nsplit != 1 && lo < hi) kv_load<HD>(ring[0], kc + cbase, vc + cbase, lo, hi - 1, lane);
  SplitStateM<HD, G> ss;
  attn_run_m<HD, G, attn_ring(HD)>(ss, qf, ring, kc + cbase, vc + cbase, lo, hi, scale, lane);

  const long hbase = (long)r * Hq + kh * G;
  if (nsplit == 1) {
    attn_store_o_m<HD, G>(ss, o + hbase * HD, lane);
  } else if (n < G) {
    // head n's partial: lane (n, grp) holds d = 128 j + 8 (4 grp + i) + b, b = 0..7
    const long pidx = (hbase + n) * nsplit + sp;
    if (grp == 0) {
      pm[pidx] = ss.m_run;
      pl[pidx] = ss.l_run;
    }
#pragma unroll
    for (int j = 0; j < NDP; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 128 * j + 8 * (4 * grp + i);
        if (d0 < HD) {
          float* dst = pa + pidx * HD + d0;
          *(f32x4*)dst = (f32x4){ss.acc[j][0][i], ss.acc[j][1][i], ss.acc[j][2][i], ss.acc[j][3][i]};
          *(f32x4*)(dst + 4) = (f32x4){ss.acc[j][4][i], ss.acc[j][5][i], ss.acc[j][6][i], ss.acc[j][7][i]};
        }
      }
  }
}

// o[rh, d] = sum_s w_s pa[rh, s, d] / sum_s w_s pl[rh, s],  w_s = exp(pm[rh, s] - max_s pm)
// with w_s = 0 for empty splits (app/kernels.py:156-167).  Every partial load of the block is
// issued before the weights are known, so the kernel costs one memory round trip.
constexpr int CMB_MAXS = 64;

// One block per (row, head), one thread per d (blockDim = HD rounded up to 64).
__global__ __launch_bounds__(512) void attn_combine_kernel(const float* __restrict__ pm,
                                                           const float* __restrict__ pl,
                                                           const float* __restrict__ pa,
                                                           f16* __restrict__ o, int HD,
                                                           int nsplit) {
  const long rh = blockIdx.x;
  const int d = threadIdx.x;
  __shared__ float s_w[CMB_MAXS];
  __shared__ float s_den;
  if (nsplit <= CMB_MAXS) {
    float av[CMB_MAXS];
#pragma unroll
    for (int sp = 0; sp < CMB_MAXS; ++sp)
      if (sp < nsplit && d < HD) av[sp] = pa[(rh * nsplit + sp) * HD + d];
    if (d < 64) {
      const float mv = d < nsplit ? pm[rh * nsplit + d] : -INFINITY;
      const float lv = d < nsplit ? pl[rh * nsplit + d] : 0.f;
      const float M = wave_max(mv);
      const float w = mv > -INFINITY ? __expf(mv - M) : 0.f;
      const float den = wave_sum(lv * w);
      if (d < nsplit) s_w[d] = w;
      if (d == 0) s_den = den;
    }
    __syncthreads();
    if (d < HD) {
      float acc = 0.f;
#pragma unroll
      for (int sp = 0; sp < CMB_MAXS; ++sp)
        if (sp < nsplit) acc += av[sp] * s_w[sp];
      o[rh * HD + d] = (f16)(acc / s_den);
    }
    return;
  }
  // many splits: plain loops
  const float* mrow = pm + rh * nsplit;
  const float* lrow = pl + rh * nsplit;
  float M = -INFINITY;
  for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, mrow[sp]);
  float den = 0.f;
  for (int sp = 0; sp < nsplit; ++sp) {
    const float m = mrow[sp];
    den += lrow[sp] * (m > -INFINITY ? __expf(m - M) : 0.f);
  }
  if (d < HD) {
    float a = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float m = mrow[sp];
      a += pa[(rh * nsplit + sp) * HD + d] * (m > -INFINITY ? __expf(m - M) : 0.f);
    }
    o[rh * HD + d] = (f16)(a / den);
  }
}

// Short caches (the depth decoder's, at most SHORT_L slots) with one split: one wave per (kv
// head, row) on the VALU, no tiles (short_attn_wave: lane l owns dims [DPL l, DPL l + DPL) of
// every head, DPL = HD / 64).  All LT >= L slots of the cache (slot indices clamped to L - 1),
// q and the position are loaded at once (one memory round trip).  Only the summation order
// differs from the tiled kernel.
constexpr int SHORT_L = 16;

template <int HD, int G, int LT>
__global__ __launch_bounds__(64) void short_attn_kernel(
    const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
    const int64_t* __restrict__ pos, f16* __restrict__ o, int S, int Hq, int Hk, int L,
    float scale) {
  static_assert(HD % 128 == 0 && HD <= 512, "an even number of dims per lane");
  constexpr int DPL = HD / 64;  // dims per lane
  constexpr int NW = DPL / 2;   // 32-bit words per lane of one row
  const int lane = threadIdx.x;
  const int kh = blockIdx.x, r = blockIdx.y;
  const long cbase = ((long)(r / S) * Hk + kh) * (long)L * HD + DPL * lane;
  uint32_t kw[LT][NW], vw[LT][NW], qw[G][NW];
#pragma unroll
  for (int t = 0; t < LT; ++t) {
    const long off = cbase + (long)min(t, L - 1) * HD;
    const uint32_t* kp = (const uint32_t*)(kc + off);
    const uint32_t* vp = (const uint32_t*)(vc + off);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      kw[t][w] = kp[w];
      vw[t][w] = vp[w];
    }
  }
  const long hb = (long)r * Hq + kh * G;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint32_t* qp = (const uint32_t*)(q + (hb + g) * HD + DPL * lane);
#pragma unroll
    for (int w = 0; w < NW; ++w) qw[g][w] = qp[w];
  }
  const long praw = pos[r];
  const int n = (int)(praw + 1 < 0 ? 0 : (praw + 1 > L ? L : praw + 1));  // slots [0, n)
  short_attn_wave<HD, G, LT>(kw, vw, qw, n, scale, o + hb * HD + DPL * lane);
}

template <int HD, int LT>
static int launch_short_l(int G, dim3 grid, hipStream_t st, const f16* q, const f16* kc,
                          const f16* vc, const int64_t* pos, f16* o, int S, int Hq, int Hk,
                          int L, float scale) {
#define ECD_SHORT_G(G_)                                                                         \
  case G_:                                                                                      \
    hipLaunchKernelGGL((short_attn_kernel<HD, G_, LT>), grid, dim3(64), 0, st, q, kc, vc, pos, o, \
                       S, Hq, Hk, L, scale);                                                    \
    return ECD_OK;
  switch (G) {
    ECD_SHORT_G(1)
    ECD_SHORT_G(2)
    ECD_SHORT_G(3)
    ECD_SHORT_G(4)
    default:
      return ECD_ENOTSUP;
  }
#undef ECD_SHORT_G
}

template <int HD>
static int launch_short(int G, dim3 grid, hipStream_t st, const f16* q, const f16* kc,
                        const f16* vc, const int64_t* pos, f16* o, int S, int Hq, int Hk, int L,
                        float scale) {
  if (L <= 8) return launch_short_l<HD, 8>(G, grid, st, q, kc, vc, pos, o, S, Hq, Hk, L, scale);
  return launch_short_l<HD, SHORT_L>(G, grid, st, q, kc, vc, pos, o, S, Hq, Hk, L, scale);
}

template <int HD>
static int launch_hd(int G, dim3 grid, hipStream_t st, const f16* q, const f16* kc,
                     const f16* vc, const int64_t* pos, f16* o, float* pm, float* pl, float* pa,
                     int S, int Hq, int Hk, int L, float scale, int nsplit) {
#define ECD_ATTN_G(G_)                                                                    \
  case G_:                                                                                \
    hipLaunchKernelGGL((decode_attn_kernel<HD, G_>), grid, dim3(64), 0, st, q, kc, vc, pos, o, \
                       pm, pl, pa, S, Hq, Hk, L, scale, nsplit);                          \
    return ECD_OK;
  switch (G) {
    ECD_ATTN_G(1)
    ECD_ATTN_G(2)
    ECD_ATTN_G(3)
    ECD_ATTN_G(4)
    ECD_ATTN_G(6)
    ECD_ATTN_G(8)
    default:
      return ECD_ENOTSUP;
  }
#undef ECD_ATTN_G
}

// ---- The split attention and its merge in one launch (the engine's attention over long caches).
// A workgroup of MW waves takes MW consecutive splits of one (row, kv head) pair (wave w: split
// MW kb + w of the pair's KB MW), runs them as decode_attn_kernel does, and merges its waves'
// partials in LDS by log-sum-exp in wave order.  Its partial (m, l, acc of each query head) goes
// to the workspace with agent-scope stores (written through to memory); once they are
// acknowledged, the workgroup counts itself on the pair's counter (an agent-scope atomic).  The
// workgroup that brings the count to KB merges the KB partials in order (agent-scope loads, so
// no stale L2 line of another XCD's partial is read) into o and resets the counter, which is
// zero again for the next call.  No workgroup waits for another: any residency is safe.  The
// merge steps are those of attn_combine_kernel: M = max m, w = exp(m - M) (0 for empty parts),
// o = fp16(sum w acc / sum w l), applied twice (waves, then workgroups).
constexpr int MW = 8;        // waves (splits) per workgroup
constexpr int MKB_MAX = 32;  // workgroups per pair at most

__device__ __forceinline__ void st_agent_f32(float* p, float v) {
  __hip_atomic_store((uint32_t*)p, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent_f32(const float* p) {
  return __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}

template <int HD, int G>
__global__ __launch_bounds__(64 * MW) void decode_attn_merged_kernel(
    const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
    const int64_t* __restrict__ pos, f16* __restrict__ o, float* __restrict__ ws,
    uint32_t* __restrict__ cnt, int S, int Hq, int Hk, int L, float scale) {
  constexpr int NDP = SplitStateM<HD, G>::NDP;
  constexpr int PS = 2 + HD;  // floats of one head's partial: m, l, acc[HD]
  __shared__ float part[MW][G][PS];
  __shared__ float s_m[MKB_MAX][G];
  __shared__ float s_l[MKB_MAX][G];
  __shared__ uint32_t s_last;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kb = blockIdx.x, KB = gridDim.x, kh = blockIdx.y, r = blockIdx.z;
  const long cbase = ((long)(r / S) * Hk + kh) * (long)L * HD;

  KVTile<HD> ring[attn_ring(HD)];
  f16x8 qf[HD / 32];
  load_q<HD, G>(qf, q, r, Hq, kh, lane);
  int lo, hi;
  split_range(pos, r, L, KB * MW, kb * MW + wv, lo, hi);
  if (lo < hi) kv_load<HD>(ring[0], kc + cbase, vc + cbase, lo, hi - 1, lane);
  SplitStateM<HD, G> ss;
  attn_run_m<HD, G, attn_ring(HD)>(ss, qf, ring, kc + cbase, vc + cbase, lo, hi, scale, lane);

  // the wave's partial to LDS: lane (n, grp) holds head n's d = 128 j + 8 (4 grp + i) + b
  const int n = lane & 15, grp = lane >> 4;
  if (n < G) {
    float* pp = part[wv][n];
    if (grp == 0) {
      pp[0] = ss.m_run;
      pp[1] = ss.l_run;
    }
#pragma unroll
    for (int j = 0; j < NDP; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 128 * j + 8 * (4 * grp + i);
        if (d0 < HD)
#pragma unroll
          for (int b = 0; b < 8; ++b) pp[2 + d0 + b] = ss.acc[j][b][i];
      }
  }
  __syncthreads();

  // the workgroup's partial: thread t merges item (g, d) over the MW waves
  const long pair = (long)r * Hk + kh;
  float* wsp = ws + pair * KB * G * PS;  // [KB][G][PS] of this pair
  for (int it = threadIdx.x; it < G * HD; it += 64 * MW) {
    const int g = it / HD, d = it - g * HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < MW; ++w) M = fmaxf(M, part[w][g][0]);
    float a = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < MW; ++w) {
      const float m = part[w][g][0];
      const float wt = m > -INFINITY ? __expf(m - M) : 0.f;
      a += part[w][g][2 + d] * wt;
      l += part[w][g][1] * wt;
    }
    float* dst = wsp + ((long)kb * G + g) * PS;
    st_agent_f32(dst + 2 + d, a);
    if (d == 0) {
      st_agent_f32(dst, M);
      st_agent_f32(dst + 1, l);
    }
  }
  wait_vm0();  // this thread's partial stores are acknowledged
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(cnt + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(KB - 1);
  __syncthreads();
  if (!s_last) return;

  // the pair's last workgroup: merge the KB partials in order
  if (threadIdx.x < KB * G) {
    const int k = threadIdx.x / G, g = threadIdx.x - k * G;
    s_m[k][g] = ld_agent_f32(wsp + ((long)k * G + g) * PS);
    s_l[k][g] = ld_agent_f32(wsp + ((long)k * G + g) * PS + 1);
  }
  __syncthreads();
  for (int it = threadIdx.x; it < G * HD; it += 64 * MW) {
    const int g = it / HD, d = it - g * HD;
    float av[MKB_MAX];
#pragma unroll
    for (int k = 0; k < MKB_MAX; ++k)
      av[k] = k < KB ? ld_agent_f32(wsp + ((long)k * G + g) * PS + 2 + d) : 0.f;
    float M = -INFINITY;
    for (int k = 0; k < KB; ++k) M = fmaxf(M, s_m[k][g]);
    float a = 0.f, den = 0.f;
#pragma unroll
    for (int k = 0; k < MKB_MAX; ++k) {
      if (k < KB) {
        const float m = s_m[k][g];
        const float wt = m > -INFINITY ? __expf(m - M) : 0.f;
        a += av[k] * wt;
        den += s_l[k][g] * wt;
      }
    }
    o[((long)r * Hq + kh * G + g) * HD + d] = (f16)(a / den);
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD>
static int launch_merged(int G, dim3 grid, hipStream_t st, const f16* q, const f16* kc,
                         const f16* vc, const int64_t* pos, f16* o, float* ws, uint32_t* cnt,
                         int S, int Hq, int Hk, int L, float scale) {
#define ECD_MERGED_G(G_)                                                                      \
  case G_:                                                                                    \
    hipLaunchKernelGGL((decode_attn_merged_kernel<HD, G_>), grid, dim3(64 * MW), 0, st, q, kc, \
                       vc, pos, o, ws, cnt, S, Hq, Hk, L, scale);                             \
    return ECD_OK;
  switch (G) {
    ECD_MERGED_G(1)
    ECD_MERGED_G(2)
    ECD_MERGED_G(3)
    ECD_MERGED_G(4)
    ECD_MERGED_G(8)
    default:
      return ECD_ENOTSUP;
  }
#undef ECD_MERGED_G
}

// Split partials of ecd_decode_attn_noalloc, for callers that cannot allocate: one static
// array per GPU (each device holds its own copy at its own address), laid out as the
// caller-supplied pm | pl | pa of ecd_decode_attn.  Every used slot is written by the attention
// kernel before the combine reads it (empty splits write m = -inf, l = 0, acc = 0), so nothing
// is cleared between calls; calls that overlap on one GPU share the array and race.
constexpr long ATTN_SCRATCH_BYTES = 8l << 20;
static __device__ __align__(256) unsigned char attn_scratch[ATTN_SCRATCH_BYTES];

// Device address of attn_scratch on the current device, looked up once per device with that
// device current (host code must never pass the array's name itself to a kernel).
constexpr int SCRATCH_MAX_DEVICES = 64;
static void* g_scratch_ptr[SCRATCH_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int attn_scratch_ptr(void** out, hipStream_t st) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return ECD_ENOTSUP;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the lookup may load the code object on this device: not while `st` is being captured
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return (int)e;
    if (cs != hipStreamCaptureStatusNone) return ECD_ENOTSUP;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(attn_scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return ECD_ENOTSUP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ECD_OK;
}

}  // namespace ecd

using namespace ecd;

extern "C" {

int ecd_decode_attn(const void* q, const void* kc, const void* vc, const int64_t* pos, void* o,
                    float* pm, float* pl, float* pa, int R, int S, int Hq, int Hk, int L, int HD,
                    int nsplit, float scale, void* stream) {
  if (!q || !kc || !vc || !pos || R <= 0 || S <= 0 || Hq <= 0 || Hk <= 0 || L <= 0 || HD <= 0 ||
      nsplit <= 0 || (Hq % Hk) != 0)
    return ECD_EINVAL;
  if (nsplit == 1 && !o) return ECD_EINVAL;
  if (nsplit > 1 && (!pm || !pl || !pa)) return ECD_EINVAL;
  const int G = Hq / Hk;
  dim3 grid(nsplit, Hk, R);
  hipStream_t st = (hipStream_t)stream;
  const f16 *qh = (const f16*)q, *kh = (const f16*)kc, *vh = (const f16*)vc;
  f16* oh = (f16*)o;
  int rc;
  // one split over a short cache: the VALU kernel (one memory round trip, no tiles)
  if (nsplit == 1 && L <= SHORT_L && G <= 4 && (HD == 128 || HD == 256 || HD == 384)) {
    const dim3 sg(Hk, R);
    rc = HD == 128   ? launch_short<128>(G, sg, st, qh, kh, vh, pos, oh, S, Hq, Hk, L, scale)
         : HD == 256 ? launch_short<256>(G, sg, st, qh, kh, vh, pos, oh, S, Hq, Hk, L, scale)
                     : launch_short<384>(G, sg, st, qh, kh, vh, pos, oh, S, Hq, Hk, L, scale);
    if (rc != ECD_OK) return rc;
    return ecd_launch_status();
  }
  switch (HD) {
    case 64:
      rc = launch_hd<64>(G, grid, st, qh, kh, vh, pos, oh, pm, pl, pa, S, Hq, Hk, L, scale, nsplit);
      break;
    case 128:
      rc = launch_hd<128>(G, grid, st, qh, kh, vh, pos, oh, pm, pl, pa, S, Hq, Hk, L, scale, nsplit);
      break;
    case 256:
      rc = launch_hd<256>(G, grid, st, qh, kh, vh, pos, oh, pm, pl, pa, S, Hq, Hk, L, scale, nsplit);
      break;
    case 384:
      rc = launch_hd<384>(G, grid, st, qh, kh, vh, pos, oh, pm, pl, pa, S, Hq, Hk, L, scale, nsplit);
      break;
    default:
      rc = ECD_ENOTSUP;
  }
  if (rc != ECD_OK) return rc;
  return ecd_launch_status();
}

int ecd_decode_attn_noalloc(const void* q, const void* kc, const void* vc, const int64_t* pos,
                            void* o, int R, int S, int Hq, int Hk, int L, int HD, int nsplit,
                            float scale, void* stream) {
  if (!q || !kc || !vc || !pos || !o || R <= 0 || S <= 0 || Hq <= 0 || Hk <= 0 || L <= 0 ||
      HD <= 0 || HD > 512 || nsplit <= 0 || (Hq % Hk) != 0)
    return ECD_EINVAL;
  if (nsplit == 1)
    return ecd_decode_attn(q, kc, vc, pos, o, nullptr, nullptr, nullptr, R, S, Hq, Hk, L, HD, 1,
                           scale, stream);
  // pm [RHs] | pl [RHs] | pa [RHs, HD] fp32, RHs = R * Hq * nsplit, each part 256-byte aligned
  const long rhs = (long)R * Hq * nsplit;
  const long part = ((rhs * 4 + 255) / 256) * 256;
  const long need = 2 * part + rhs * HD * 4;
  if (need > ATTN_SCRATCH_BYTES) return ECD_ENOMEM;
  void* base = nullptr;
  const int rc = attn_scratch_ptr(&base, (hipStream_t)stream);
  if (rc != ECD_OK) return rc;
  float* pm = (float*)base;
  float* pl = (float*)((char*)base + part);
  float* pa = (float*)((char*)base + 2 * part);
  const int r1 = ecd_decode_attn(q, kc, vc, pos, o, pm, pl, pa, R, S, Hq, Hk, L, HD, nsplit, scale,
                                 stream);
  if (r1 != ECD_OK) return r1;
  return ecd_attn_combine(pm, pl, pa, o, R * Hq, HD, nsplit, stream);
}

int ecd_decode_attn_merged(const void* q, const void* kc, const void* vc, const int64_t* pos,
                           void* o, float* ws, uint32_t* cnt, int R, int S, int Hq, int Hk, int L,
                           int HD, int kb, float scale, void* stream) {
  if (!q || !kc || !vc || !pos || !o || !ws || !cnt || R <= 0 || S <= 0 || Hq <= 0 || Hk <= 0 ||
      L <= 0 || HD <= 0 || (Hq % Hk) != 0 || kb < 1 || kb > MKB_MAX || (long)R * Hk > 65535)
    return ECD_EINVAL;
  const int G = Hq / Hk;
  const dim3 grid(kb, Hk, R);
  hipStream_t st = (hipStream_t)stream;
  const f16 *qh = (const f16*)q, *kh = (const f16*)kc, *vh = (const f16*)vc;
  f16* oh = (f16*)o;
  int rc;
  switch (HD) {
    case 128:
      rc = launch_merged<128>(G, grid, st, qh, kh, vh, pos, oh, ws, cnt, S, Hq, Hk, L, scale);
      break;
    case 256:
      rc = launch_merged<256>(G, grid, st, qh, kh, vh, pos, oh, ws, cnt, S, Hq, Hk, L, scale);
      break;
    case 384:
      rc = launch_merged<384>(G, grid, st, qh, kh, vh, pos, oh, ws, cnt, S, Hq, Hk, L, scale);
      break;
    default:
      rc = ECD_ENOTSUP;
  }
  if (rc != ECD_OK) return rc;
  return ecd_launch_status();
}

int ecd_attn_combine(const float* pm, const float* pl, const float* pa, void* o, int RH, int HD,
                     int nsplit, void* stream) {
  if (!pm || !pl || !pa || !o || RH <= 0 || HD <= 0 || HD > 512 || nsplit <= 0) return ECD_EINVAL;
  const int threads = ((HD + 63) / 64) * 64;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(RH), dim3(threads), 0, (hipStream_t)stream, pm, pl,
                     pa, (f16*)o, HD, nsplit);
  return ecd_launch_status();
}

}  // extern "C"
