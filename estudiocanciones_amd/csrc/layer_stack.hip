// C entry points of the layer-stack launch (the kernels: layer_tail.h).  Compiled on its own, with
// machine loop-invariant code motion off: hoisted out of the layer loop, constants and addresses
// would be held in registers across all of it, which the 3072-wide stacks do not have.
#include "layer_tail.h"

using namespace ecd;

// Backbone layers per launch, unrolled: 28 layers as 4 launches (measured against 2 and 4 layers
// per launch: 557.8 / 561.2 / 563.1 frames/s at KV 750; 14 per launch adds 0.1% for twice the
// code and build time).
constexpr int BB_NLU = 7;

// Stack launches: the instantiated shapes.  The depth decoders take all their layers in one
// launch; the backbone takes BB_NLU layers per launch, unrolled (looped over its layers, its
// 3072-wide tail with the MFMA attention needs more than the 168 registers a lane has at three
// waves per SIMD).  0: not instantiated, else an index for ecd_layer_stack's dispatch.
static int stack_kind(int nb, int M, int D, int F, int Hq, int Hk, int HD, int L, bool ntl, bool knt) {
  if (nb <= 0 || (nb % 8) || M < 1 || M > tail::MR || Hk <= 0 || (Hq % Hk) || D <= 0 ||
      (D % 512) || F != 8192 || !tail_att_ok(nb, M, D, Hq, Hk, HD, L))
    return 0;
  const int cd = D / 64 / tail::CW, ag = Hq / Hk, rt = M > 8 ? 16 : 8;
  const bool vs = L <= tail::VSHORT;
  const int ks2 = (nb % (D / 16) == 0 && nb / (D / 16) == 4) ? 4 : 1;
  if (2 * F / 16 != 4 * nb || (Hq + 2 * Hk) * HD / 16 > 2 * nb) return 0;
  // the backbone: 3072 wide, 24q / 8kv, head_dim 128, streamed weights, up to 8 rows
  if (cd == 6 && ks2 == 1 && HD == 128 && ag == 3 && rt == 8 && !vs && ntl) return knt ? 2 : 1;
  // the reference depth decoder: 3072 wide, 8q / 4kv, head_dim 384, 8-slot caches
  if (cd == 6 && ks2 == 1 && HD == 384 && ag == 2 && vs && !ntl && !knt) return rt == 8 ? 3 : 4;
  // the 1024-wide depth decoder: 8q / 2kv, head_dim 128, 8-slot caches
  if (cd == 2 && ks2 == 4 && HD == 128 && ag == 4 && vs && !ntl && !knt) return rt == 8 ? 5 : 6;
  return 0;
}

extern "C" int ecd_layer_stack_supported(int nl, int M, int D, int F, int Hq, int Hk, int HD,
                                         int L, int flags) {
  const int kind = stack_kind(tail::device_cus(), M, D, F, Hq, Hk, HD, L, (flags >> 1) & 1,
                              (flags >> 3) & 1);
  // the backbone's launches take BB_NLU layers each
  if (nl < 1 || nl > ECD_STACK_MAX || ((kind == 1 || kind == 2) && nl % BB_NLU)) return ECD_ENOTSUP;
  switch (kind) {
    case 1: return tail::stack_scratch_free<6, 16, 4, 1, 128, 3, true, 8, false, false, BB_NLU>() ? ECD_OK : ECD_ENOTSUP;
    case 2: return tail::stack_scratch_free<6, 16, 4, 1, 128, 3, true, 8, false, true, BB_NLU>() ? ECD_OK : ECD_ENOTSUP;
    case 3: return tail::stack_scratch_free<6, 16, 4, 1, 384, 2, false, 8, true, false>() ? ECD_OK : ECD_ENOTSUP;
    case 4: return tail::stack_scratch_free<6, 16, 4, 1, 384, 2, false, 16, true, false>() ? ECD_OK : ECD_ENOTSUP;
    case 5: return tail::stack_scratch_free<2, 16, 4, 4, 128, 4, false, 8, true, false>() ? ECD_OK : ECD_ENOTSUP;
    case 6: return tail::stack_scratch_free<2, 16, 4, 4, 128, 4, false, 16, true, false>() ? ECD_OK : ECD_ENOTSUP;
  }
  return ECD_ENOTSUP;
}

extern "C" int ecd_layer_stack_layers_per_launch(int nl, int M, int D, int F, int Hq, int Hk,
                                                 int HD, int L, int flags) {
  if (ecd_layer_stack_supported(nl, M, D, F, Hq, Hk, HD, L, flags) != ECD_OK) return ECD_ENOTSUP;
  const int kind = stack_kind(tail::device_cus(), M, D, F, Hq, Hk, HD, L, (flags >> 1) & 1,
                              (flags >> 3) & 1);
  return kind == 1 || kind == 2 ? BB_NLU : nl;
}

extern "C" long ecd_layer_stack_plan_bytes(int nl) {
  return nl > 0 ? (long)nl * (long)sizeof(tail::LayerRec) : 0;
}

extern "C" int ecd_layer_stack_plan(const void* layers, int nl, int M, int D, int F, int Hq, int Hk,
                                    int HD, int yld, void* plan, void* stream) {
  static_assert(sizeof(tail::LayerRec) == 17 * sizeof(void*), "17 pointers per layer");
  if (!layers || !plan || nl < 1 || nl > ECD_STACK_MAX || M < 1 || M > tail::MR || D <= 0 ||
      F <= 0 || Hq <= 0 || Hk <= 0 || HD <= 0 || yld < 0 || ((uintptr_t)plan & 15))
    return ECD_EINVAL;
  const tail::LayerRec* r = (const tail::LayerRec*)layers;
  auto al = [](const void* p) { return p && ((uintptr_t)p & 15) == 0; };
  auto apart = [](const void* p, long pb, const void* q, long qb) {
    const uintptr_t a = (uintptr_t)p, c = (uintptr_t)q;
    return a + pb <= c || c + qb <= a;
  };
  const long bx = 2L * M * D, bm = 2L * M * F, bo = 2L * M * Hq * HD, by = 2L * M * yld;
  for (int l = 0; l < nl; ++l) {
    const tail::LayerRec& e = r[l];
    if (!al(e.wo) || !e.so || !al(e.n2) || !al(e.w13) || !e.s13 || !al(e.w2) || !e.s2 ||
        !al(e.x1) || !al(e.mm) || !al(e.xout))
      return ECD_EINVAL;
    // every layer but the last runs the next layer's q|k|v and attention (its o_next is the
    // next layer's o); the last may or may not, or may end in a codebook head (y: the 1024-wide
    // decoder only, wq / sq / n1 the head's weights and norm, no caches or attention)
    const bool nxt = e.wq != nullptr;
    if (e.y) {
      if (l + 1 < nl || D != 1024 || yld <= 0 || !al(e.y) || !al(e.n1) || !al(e.wq) || !e.sq || e.kc ||
          e.vc || e.o_next)
        return ECD_EINVAL;
    } else {
      if (l + 1 < nl && (!nxt || !e.o_next)) return ECD_EINVAL;
      if (nxt && (!al(e.n1) || !al(e.wq) || !e.sq || !e.kc || !e.vc || !al(e.o_next)))
        return ECD_EINVAL;
      if (!nxt && e.o_next) return ECD_EINVAL;
    }
    // a layer's outputs are its own: no two of x1, mm, xout, o_next, y overlap, here or in any
    // other layer of the stack
    const void* out[5] = {e.x1, e.mm, e.xout, e.o_next, e.y};
    const long ob[5] = {bx, bm, bx, bo, by};
    for (int k = 0; k <= l; ++k) {
      const tail::LayerRec& f = r[k];
      const void* o2[5] = {f.x1, f.mm, f.xout, f.o_next, f.y};
      for (int i = 0; i < 5; ++i)
        for (int j = 0; j < 5; ++j) {
          if (k == l && j <= i) continue;
          if (out[i] && o2[j] && !apart(out[i], ob[i], o2[j], ob[j])) return ECD_EINVAL;
        }
    }
  }
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(plan, layers, (size_t)nl * sizeof(tail::LayerRec),
                                hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  return e == hipSuccess ? ECD_OK : (int)e;
}

extern "C" int ecd_layer_stack(const void* plan, int nl, const void* o, const void* xin,
                               const float* rope, const int64_t* pos, void* q, void* sync,
                               void* err, void* ws, int M, int D, int F, int S, int Hq, int Hk,
                               int L, int HD, int yn, int yld, float eps, int flags,
                               void* stream) {
  auto al = [](const void* p) { return p && ((uintptr_t)p & 15) == 0; };
  if (!al(plan) || nl < 1 || nl > ECD_STACK_MAX || !al(o) || !al(xin) || !rope || !pos || !q ||
      !sync || ((uintptr_t)sync & 255) || !err || !al(ws) || S <= 0 || L <= 0 || (HD % 4) ||
      yn < 0 || yld < yn)
    return ECD_EINVAL;
  const int nb = tail::device_cus();
  const bool ntl = (flags >> 1) & 1, knt = (flags >> 3) & 1;
  const int kind = stack_kind(nb, M, D, F, Hq, Hk, HD, L, ntl, knt);
  if (!kind) return ECD_ENOTSUP;
  // a codebook head in the last layer: at most three 16-column tiles per workgroup
  if (yn > 48 * nb) return ECD_ENOTSUP;
  if (L <= tail::VSHORT && S > tail::VNEW) return ECD_ENOTSUP;
  tail::Args a = {};
  a.o = (const f16*)o; a.xin = (const f16*)xin;
  a.rope = rope; a.pos = pos; a.q = (f16*)q;
  a.S = S; a.Hq = Hq; a.Hk = Hk; a.L = L; a.HD = HD;
  // attention scale: the fp32 rounding of 1 / sqrt(HD) (the reference passes it as a float)
  a.scale = (float)(1.0 / sqrt((double)HD));
  a.sync = (uint32_t*)sync; a.err = (uint32_t*)err; a.ws = (float*)ws;
  a.M = M; a.D = D; a.F = F; a.eps = eps; a.spin_max = (flags & 4) ? 0 : 1 << 17;
  a.yn = yn; a.yld = yld;
  const tail::LayerRec* pl = (const tail::LayerRec*)plan;
  hipStream_t st = (hipStream_t)stream;
  switch (kind) {
    case 1: return tail::launch_stack<6, 16, 4, 1, 128, 3, true, 8, false, false, BB_NLU>(a, pl, nl, nb, st);
    case 2: return tail::launch_stack<6, 16, 4, 1, 128, 3, true, 8, false, true, BB_NLU>(a, pl, nl, nb, st);
    case 3: return tail::launch_stack<6, 16, 4, 1, 384, 2, false, 8, true, false>(a, pl, nl, nb, st);
    case 4: return tail::launch_stack<6, 16, 4, 1, 384, 2, false, 16, true, false>(a, pl, nl, nb, st);
    case 5: return tail::launch_stack<2, 16, 4, 4, 128, 4, false, 8, true, false>(a, pl, nl, nb, st);
    case 6: return tail::launch_stack<2, 16, 4, 4, 128, 4, false, 16, true, false>(a, pl, nl, nb, st);
  }
  return ECD_ENOTSUP;
}
