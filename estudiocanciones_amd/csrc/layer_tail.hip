// C entry points of the per-layer tail and head launches (the kernels: layer_tail.h).
#include "layer_tail.h"

using namespace ecd;

extern "C" int ecd_layer_head(const void* xin, const void* n1, const void* wq, const void* sq,
                              const float* rope, const int64_t* pos, void* q, void* kc, void* vc,
                              void* o_next, void* sync, void* err, void* ws, int M, int D, int F,
                              int S, int Hq, int Hk, int L, int HD, float eps, int flags,
                              void* stream) {
  tail::Args a = {};
  a.xin = (const f16*)xin;
  a.n1 = (const f16*)n1; a.wq = (const int8_t*)wq; a.sq = (const f16*)sq;
  a.rope = rope; a.pos = pos; a.q = (f16*)q; a.kc = (f16*)kc; a.vc = (f16*)vc;
  a.S = S; a.Hq = Hq; a.Hk = Hk; a.L = L; a.HD = HD;
  // attention scale: the fp32 rounding of 1 / sqrt(HD) (the reference passes it as a float)
  a.o_next = (f16*)o_next; a.scale = HD > 0 ? (float)(1.0 / sqrt((double)HD)) : 0.f;
  a.sync = (uint32_t*)sync; a.err = (uint32_t*)err; a.ws = (float*)ws;
  a.M = M; a.D = D; a.F = F; a.eps = eps; a.spin_max = (flags & 4) ? 0 : 1 << 17;
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!xin || !n1 || !wq || !sq || !rope || !pos || !q || !kc || !vc || !o_next || !sync ||
      !err || !ws || M < 1 || M > tail::MR || D <= 0 || F <= 0 || (D % 512) || (F % 512) ||
      S <= 0 || Hq <= 0 || Hk <= 0 || (Hq % Hk) || L <= 0 || HD <= 0 || (HD % 4) ||
      (Hq + 2 * Hk) * HD % 16 || !al(xin) || !al(n1) || !al(wq) || !al(o_next) || !al(ws) ||
      ((uintptr_t)sync & 255))
    return ECD_EINVAL;
  const int nb = tail::device_cus();
  const int cd = D / 64 / tail::CW, cf = F / 64 / tail::CW;
  const int t13 = 2 * F / 16;
  if (nb <= 0 || (nb % 8) || D / 16 > nb || t13 % nb) return ECD_ENOTSUP;
  if ((Hq + 2 * Hk) * HD / 16 > 2 * nb || !tail_att_ok(nb, M, D, Hq, Hk, HD, L)) return ECD_ENOTSUP;
  const int nt13 = t13 / nb;
  const int ks2 = (nb % (D / 16) == 0 && nb / (D / 16) == 4) ? 4 : 1;
  const int ag = Hq / Hk;
  const int rt = M > 8 ? 16 : 8;  // rows of the x tile
  const bool ntl = (flags >> 1) & 1;
  const bool vs = L <= tail::VSHORT;  // the VALU attention path
  if (vs && S > tail::VNEW) return ECD_ENOTSUP;
  const bool knt = (flags >> 3) & 1;  // nontemporal cache-slot loads for every split
  hipStream_t st = (hipStream_t)stream;
#define ECD_HEAD(CD_, CF_, NT_, KS_, AHD_, AG_, R_, VS_)                                      \
  if (cd == CD_ && cf == CF_ && nt13 == NT_ && ks2 == KS_ && HD == AHD_ && ag == AG_ &&       \
      rt == R_ && vs == VS_)                                                                  \
    return ntl ? tail::launch<CD_, CF_, NT_, KS_, AHD_, AG_, true, true, R_, VS_>(a, nb, st)  \
               : tail::launch<CD_, CF_, NT_, KS_, AHD_, AG_, false, true, R_, VS_>(a, nb, st);
  if (knt && cd == 6 && cf == 16 && nt13 == 4 && ks2 == 1 && HD == 128 && ag == 3 && rt == 8 &&
      !vs)
    return ntl ? tail::launch<6, 16, 4, 1, 128, 3, true, true, 8, false, true>(a, nb, st)
               : tail::launch<6, 16, 4, 1, 128, 3, false, true, 8, false, true>(a, nb, st);
  ECD_HEAD(6, 16, 4, 1, 128, 3, 8, false)
  ECD_HEAD(6, 16, 4, 1, 128, 3, 8, true)
  ECD_HEAD(6, 16, 4, 1, 384, 2, 8, true)
  ECD_HEAD(6, 16, 4, 1, 384, 2, 16, true)
  ECD_HEAD(2, 16, 4, 4, 128, 4, 8, false)
  ECD_HEAD(2, 16, 4, 4, 128, 4, 8, true)
  ECD_HEAD(2, 16, 4, 4, 128, 4, 16, false)
  ECD_HEAD(2, 16, 4, 4, 128, 4, 16, true)
#undef ECD_HEAD
  return ECD_ENOTSUP;
}

extern "C" long ecd_layer_tail_ws_bytes(int D, int Hq, int Hk, int HD) {
  const int nb = tail::device_cus();
  // the split-W2 sums (D * 64 fp32), the attention partials [NB][G][2 + HD], all as 8-byte
  // (fp32, epoch) words, then the q|k|v hand-off [MR][Hq + 2 Hk][HD] as 8-byte (2 fp16, epoch)
  // words
  const long w2 = (long)D * 512;
  const long at = Hk > 0 ? (long)nb * (Hq / Hk) * (HD + 2) * 8 : 0;
  const long hd = Hk > 0 ? (long)tail::MR * (Hq + 2 * Hk) * HD * 4 : 0;
  return w2 + at + hd;
}

extern "C" int ecd_layer_tail(const void* o, const void* xin, const void* wo, const void* so,
                              const void* n2, const void* w13, const void* s13, const void* w2,
                              const void* s2, const void* n1, const void* wq, const void* sq,
                              const float* rope, const int64_t* pos, void* q, void* kc, void* vc,
                              void* o_next, void* x1, void* mm, void* xout, void* sync, void* err,
                              void* ws, int M, int D, int F, int S, int Hq, int Hk, int L, int HD,
                              float eps, int flags, void* stream) {
  tail::Args a = {};
  a.o = (const f16*)o; a.xin = (const f16*)xin;
  a.wo = (const int8_t*)wo; a.so = (const f16*)so; a.n2 = (const f16*)n2;
  a.w13 = (const int8_t*)w13; a.s13 = (const f16*)s13;
  a.w2 = (const int8_t*)w2; a.s2 = (const f16*)s2;
  a.n1 = (const f16*)n1; a.wq = (const int8_t*)wq; a.sq = (const f16*)sq;
  a.rope = rope; a.pos = pos; a.q = (f16*)q; a.kc = (f16*)kc; a.vc = (f16*)vc;
  a.S = S; a.Hq = Hq; a.Hk = Hk; a.L = L; a.HD = HD;
  // attention scale: the fp32 rounding of 1 / sqrt(HD) (the reference passes it as a float)
  a.o_next = (f16*)o_next; a.scale = HD > 0 ? (float)(1.0 / sqrt((double)HD)) : 0.f;
  a.x1 = (f16*)x1; a.mm = (f16*)mm; a.xout = (f16*)xout;
  a.sync = (uint32_t*)sync; a.err = (uint32_t*)err; a.ws = (float*)ws;
  a.M = M; a.D = D; a.F = F; a.eps = eps; a.spin_max = (flags & 4) ? 0 : 1 << 17;
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!o || !xin || !wo || !so || !n2 || !w13 || !s13 || !w2 || !s2 || !x1 || !mm || !xout ||
      !sync || !err || M < 1 || M > tail::MR || D <= 0 || F <= 0 || (D % 512) || (F % 512) ||
      !al(o) || !al(xin) || !al(x1) || !al(mm) || !al(xout) || !al(n2) || !al(wo) ||
      !al(w13) || !al(w2) || ((uintptr_t)sync & 255))
    return ECD_EINVAL;
  if (wq && (!n1 || !sq || !rope || !pos || !q || !kc || !vc || !al(n1) || !al(wq) || S <= 0 ||
             Hq <= 0 || Hk <= 0 || (Hq % Hk) || L <= 0 || HD <= 0 || (HD % 4) ||
             (Hq + 2 * Hk) * HD % 16))
    return ECD_EINVAL;
  if (o_next && (!wq || !al(o_next) || !ws)) return ECD_EINVAL;
  const int nb = tail::device_cus();
  const int cd = D / 64 / tail::CW, cf = F / 64 / tail::CW;
  const int t13 = 2 * F / 16;
  if (nb <= 0 || (nb % 8) || D / 16 > nb || t13 % nb)
    return ECD_ENOTSUP;
  if (wq && (Hq + 2 * Hk) * HD / 16 > 2 * nb) return ECD_ENOTSUP;
  if (o_next && !tail_att_ok(nb, M, D, Hq, Hk, HD, L)) return ECD_ENOTSUP;
  const int nt13 = t13 / nb;
  // W2 has D / 16 tiles: with four times as many CUs, K is split over 4 workgroups per tile
  const int ks2 = (nb % (D / 16) == 0 && nb / (D / 16) == 4) ? 4 : 1;
  if (ks2 > 1 && (!ws || !al(ws))) return ECD_EINVAL;
  const int ag = o_next ? Hq / Hk : 0;
  const int rt = M > 8 ? 16 : 8;  // rows of the x tile
  const bool ntl = (flags >> 1) & 1;
  const bool vs = o_next && L <= tail::VSHORT;  // the VALU attention path
  if (vs && S > tail::VNEW) return ECD_ENOTSUP;
  const bool knt = (flags >> 3) & 1;  // nontemporal cache-slot loads for every split
  hipStream_t st = (hipStream_t)stream;
  if (knt && o_next && cd == 6 && cf == 16 && nt13 == 4 && ks2 == 1 && HD == 128 && ag == 3 &&
      rt == 8 && !vs)
    return ntl ? tail::launch<6, 16, 4, 1, 128, 3, true, false, 8, false, true>(a, nb, st)
               : tail::launch<6, 16, 4, 1, 128, 3, false, false, 8, false, true>(a, nb, st);
#define ECD_TAIL(CD_, CF_, NT_, KS_, AHD_, AG_, R_, VS_)                                      \
  if (cd == CD_ && cf == CF_ && nt13 == NT_ && ks2 == KS_ && (o_next ? HD : 0) == AHD_ &&      \
      ag == AG_ && rt == R_ && vs == VS_)                                                     \
    return ntl ? tail::launch<CD_, CF_, NT_, KS_, AHD_, AG_, true, false, R_, VS_>(a, nb, st) \
               : tail::launch<CD_, CF_, NT_, KS_, AHD_, AG_, false, false, R_, VS_>(a, nb, st);
  // 3072 -> 2 x 8192 -> 3072, up to 8 rows: the backbone (with its attention: 24q / 8kv,
  // head_dim 128) and the reference's depth decoder (8q / 4kv, head_dim 384, caches of 8 slots);
  // 16 rows (the reference decoder's first pass: two rows per cache) with the VALU attention
  // or none
  ECD_TAIL(6, 16, 4, 1, 128, 3, 8, false)
  ECD_TAIL(6, 16, 4, 1, 128, 3, 8, true)
  ECD_TAIL(6, 16, 4, 1, 384, 2, 8, true)
  ECD_TAIL(6, 16, 4, 1, 0, 0, 8, false)
  ECD_TAIL(6, 16, 4, 1, 384, 2, 16, true)
  ECD_TAIL(6, 16, 4, 1, 0, 0, 16, false)
  // 1024 -> 2 x 8192 -> 1024: the 1024-wide depth decoder (8q / 2kv, head_dim 128), up to 16
  // rows (its first pass: two rows per cache)
  ECD_TAIL(2, 16, 4, 4, 128, 4, 8, false)
  ECD_TAIL(2, 16, 4, 4, 128, 4, 8, true)
  ECD_TAIL(2, 16, 4, 4, 0, 0, 8, false)
  ECD_TAIL(2, 16, 4, 4, 128, 4, 16, false)
  ECD_TAIL(2, 16, 4, 4, 128, 4, 16, true)
  ECD_TAIL(2, 16, 4, 4, 0, 0, 16, false)
#undef ECD_TAIL
  return ECD_ENOTSUP;
}

// ECD_OK when ecd_layer_tail runs these shapes on the current device (with the next layer's
// attention in the launch when `attention` is set; L = cache slots), ECD_ENOTSUP otherwise
// (the caller then runs the per-op kernels).
extern "C" int ecd_layer_tail_supported(int M, int D, int F, int Hq, int Hk, int HD, int L,
                                        int attention) {
  const int nb = tail::device_cus();
  if (M < 1 || M > tail::MR || D <= 0 || F <= 0 || (D % 512) || (F % 512) || nb <= 0 || (nb % 8))
    return ECD_ENOTSUP;
  const int cd = D / 64 / tail::CW, cf = F / 64 / tail::CW, t13 = 2 * F / 16;
  const int ks2 = (nb % (D / 16) == 0 && nb / (D / 16) == 4) ? 4 : 1;
  if (D / 16 > nb || t13 % nb || cf != 16 || t13 / nb != 4 ||
      !((cd == 6 && ks2 == 1) || (cd == 2 && ks2 == 4)))
    return ECD_ENOTSUP;
  if (Hq <= 0 || Hk <= 0 || (Hq % Hk) || HD <= 0 || (HD % 4) || (Hq + 2 * Hk) * HD % 16 ||
      (Hq + 2 * Hk) * HD / 16 > 2 * nb)
    return ECD_ENOTSUP;
  if (attention && !tail_att_ok(nb, M, D, Hq, Hk, HD, L)) return ECD_ENOTSUP;
  return ECD_OK;
}
