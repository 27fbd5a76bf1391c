/*
 * ecdecode.h -- C ABI of the MI355X (gfx950) per-frame decode path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed as
 * `void* stream` (0 = the null stream).  Nothing allocates, frees or synchronises (except the
 * set-up call ecd_layer_stack_plan, which copies a plan and waits for it), so a caller may
 * capture any sequence of the other calls into one hipGraph.  Tensors are dense,
 * row-major, fp16 unless stated ("f16" below is IEEE binary16 stored as 16 bits).
 *
 * Return value: 0 on success; ECD_EINVAL (-22) for an argument rejected on the host before
 * any launch; ECD_ENOTSUP (-95) for a shape the library does not implement; a positive
 * hipError_t code if the launch itself failed.
 *
 * Reference interfaces replaced (paths relative to the EstudioCanciones repository):
 *   app/kernels.py   -- Triton kernels and their Python launchers
 *   app/engine.py    -- the engine that launches them, RoPE table, embeddings
 *   app/convert_final.py -- the offline int8 quantiser
 */
#ifndef ECDECODE_H
#define ECDECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ECD_OK 0
#define ECD_EINVAL (-22)
#define ECD_ENOTSUP (-95)
#define ECD_ENOMEM (-12) /* the call needs more than a fixed-size static workspace */

/* int8 per-output-channel GEMV / skinny GEMM with optional residual.
 * Replaces int8_mm + _gemv8 (app/kernels.py:40-54, :20-37) and its dense fallback for
 * M > 16 rows (app/kernels.py:46-49).
 *   x [M, K] f16 with row stride ldx (elements); w [N, K] int8 (K contiguous); s [N] f16;
 *   res [M, N] f16 with row stride ldr, or NULL; y [M, N] f16 with row stride ldy.
 *   dense = 0: y = f16(f32(s[n]) * sum_k x*q)          (the reference's M <= 16 path)
 *   dense = 1: y = f16(sum_k x * f16(f16(q) * s[n]))   (the reference's M > 16 path)
 *   then y = f16(y + res) when res is given. */
int ecd_gemv_i8(const void* x, long ldx, const void* w, const void* s, const void* res, long ldr,
                void* y, long ldy, int M, int N, int K, int dense, void* stream);

/* Same as ecd_gemv_i8 with an explicit tile choice (nt = 16-row tiles per block,
 * kw = waves splitting K; 0 = library default).  Replaces the autotuned launch
 * parameters of _gemv8 (app/kernels.py:12-19). */
int ecd_gemv_i8_tuned(const void* x, long ldx, const void* w, const void* s, const void* res,
                      long ldr, void* y, long ldy, int M, int N, int K, int dense, int nt, int kw,
                      void* stream);

/* RMSNorm: y = f16(f16(x * inv) * w), inv = 1/sqrt(sum(x^2)/D + eps).
 * Replaces rms/_rms (app/kernels.py:58-74); torch twin app/engine.py:56-58.
 *   x [R, D] stride ldx, w [D], y [R, D] stride ldy. */
int ecd_rmsnorm(const void* x, long ldx, const void* w, void* y, long ldy, int R, int D,
                float eps, void* stream);

/* Interleaved RoPE of the q and k heads of a fused qkv row plus the KV-cache write.
 * Replaces _rope_cache (app/kernels.py:78-107) as launched at app/engine.py:191-192.
 *   qkv [R, (Hq + 2Hk) * HD]; rope [>= L, HD/2, 2] f32 (cos, sin); pos [R] int64;
 *   q [R, Hq * HD] (output); kc, vc [B, Hk, L, HD] written at [r / S, kh, pos[r], :].
 *   A row whose pos is outside [0, L) writes no cache slot. */
int ecd_rope_kv_write(const void* qkv, const float* rope, const int64_t* pos, void* q, void* kc,
                      void* vc, int R, int S, int Hq, int Hk, int L, int HD, void* stream);

/* GQA flash-decoding attention of each row over cache slots [0, pos[r]].
 * Replaces _attn (app/kernels.py:111-153) as launched at app/engine.py:194-202.
 *   q [R, Hq * HD]; kc, vc [B, Hk, L, HD]; pos [R] int64.
 *   nsplit == 1: writes o [R, Hq * HD] directly (pm/pl/pa unused, may be NULL).
 *   nsplit  > 1: writes partials pm, pl [R * Hq * nsplit] f32 and pa [R * Hq * nsplit, HD] f32
 *                indexed (r * Hq + h) * nsplit + split, for ecd_attn_combine.
 *   HD in {64, 128, 256, 384}; Hq / Hk in {1, 2, 3, 4, 6, 8}. */
int ecd_decode_attn(const void* q, const void* kc, const void* vc, const int64_t* pos, void* o,
                    float* pm, float* pl, float* pa, int R, int S, int Hq, int Hk, int L, int HD,
                    int nsplit, float scale, void* stream);

/* Log-sum-exp merge of the split partials into o [RH, HD] f16 (RH = R * Hq).
 * Replaces _attn_combine (app/kernels.py:156-167), launched at app/engine.py:204. */
int ecd_attn_combine(const float* pm, const float* pl, const float* pa, void* o, int RH, int HD,
                     int nsplit, void* stream);

/* ecd_decode_attn followed by ecd_attn_combine into o, with the split partials kept in a
 * static device array of 8 MiB (one per GPU) instead of caller buffers: nothing is allocated
 * on any call.  No counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under hipGraph capture that may not call hipMalloc, tight serving loops).
 * Same arguments and results as the two calls it replaces (bit for bit).  Returns ECD_ENOMEM
 * when 2 * ceil256(4 * R * Hq * nsplit) + 4 * R * Hq * nsplit * HD bytes exceed 8 MiB (e.g.
 * R = 16, Hq = 24, nsplit = 16, HD = 128 needs 3.2 MB).  The array keeps the last call's
 * contents; calls that overlap on one GPU (two streams at once) race on it.  The first call
 * with nsplit > 1 on a device looks the array's address up (hipGetSymbolAddress, which may
 * load the code object) and must not be made while `stream` is being captured: it then
 * returns ECD_ENOTSUP; later calls on that device may be captured into a hipGraph. */
int ecd_decode_attn_noalloc(const void* q, const void* kc, const void* vc, const int64_t* pos,
                            void* o, int R, int S, int Hq, int Hk, int L, int HD, int nsplit,
                            float scale, void* stream);

/* The split decode attention and its merge in one launch: the pair (_attn, _attn_combine) of
 * app/kernels.py:110-167 as launched at app/engine.py:194-204, for the engine's own attention
 * over long caches.  Grid (kb, Hk, R) of 8-wave workgroups: each (row, kv head) pair is cut
 * into 8 kb splits (chunks as in ecd_decode_attn), a workgroup merges its 8 waves' partials,
 * and the pair's last workgroup to finish merges the kb workgroup partials into o (the
 * log-sum-exp steps of ecd_attn_combine, applied per workgroup and then across them, so only
 * the fp32 summation order differs from the pair of launches).
 *   ws: [R * Hk * kb * (Hq / Hk) * (2 + HD)] f32 workgroup partials (any contents);
 *   cnt: [R * Hk] uint32 pair counters, zero before the first call; every call leaves them
 *   zero.  Two calls that run at the same time must not share ws or cnt.
 *   1 <= kb <= 32; HD in {128, 256, 384}; Hq / Hk in {1, 2, 3, 4, 8}; R * Hk <= 65535. */
int ecd_decode_attn_merged(const void* q, const void* kc, const void* vc, const int64_t* pos,
                           void* o, float* ws, uint32_t* cnt, int R, int S, int Hq, int Hk, int L,
                           int HD, int kb, float scale, void* stream);

/* y[r, c] = f16(f16(silu(x[r, c])) * x[r, F + c]) for x [R, 2F], y [R, F].
 * Replaces _silu_mul (app/kernels.py:171-180), launched at app/engine.py:209. */
int ecd_silu_mul(const void* x, void* y, int R, int F, void* stream);

/* Backbone input: out[b] = f16(sum_c f16(f16(q[row]) * s[row])), row = tok[b, c] + c * vocab.
 * Replaces Emb.__call__ + .sum(1, dtype) (app/engine.py:89-104, :348).
 *   tok [B, C] int64; table [rows, D] int8; scales [rows] f16; out [B, D].  A token outside
 *   [0, vocab), or whose row is >= rows, contributes nothing. */
int ecd_embed_sum_i8(const int64_t* tok, const void* table, const void* scales, long rows,
                     void* out, int B, int C, int D, int vocab, void* stream);

/* One-codebook embedding: e[b] = f16(f16(q[row]) * s[row]), row = tok[b * tok_stride] + cb * vocab
 * (zero for a token outside [0, vocab) or a row >= rows; table [rows, D], scales [rows]).
 * even == NULL: out[b] = e[b] (out [B, D]).
 * even != NULL: out[2b] = even[b], out[2b + 1] = e[b] (out [2B, D]), the two-row input of the
 *               first decoder pass.
 * Replaces _embed_audio (app/engine.py:307-308) and the stack at app/engine.py:336. */
int ecd_embed_i8(const int64_t* tok, long tok_stride, const void* table, const void* scales,
                 long rows, int cb, int vocab, const void* even, void* out, int B, int D,
                 void* stream);

/* Per-row symmetric int8 quantiser of w [N, K] f32: s = max(max|w|, 1e-8) / 127,
 * q = clamp(round_half_even(w / s), -127, 127); s_bf16 [N] (bf16 bits, nearest even) and/or
 * s_f16 [N] (the f16 value of that bf16) -- either may be NULL, not both.
 * Replaces q8_rows (app/convert_final.py:17-21) and the load cast at app/engine.py:241. */
int ecd_quantize_rows_i8(const float* w, void* q, void* s_bf16, void* s_f16, int N, int K,
                         void* stream);

/* Llama-3 scaled RoPE table out [max_seq, head_dim / 2, 2] f32 (cos, sin), on the device.
 * Replaces rope_cache (app/engine.py:28-43) built at Stack.alloc (app/engine.py:165-166). */
int ecd_rope_table(float* out, int max_seq, int head_dim, double base, double scale, double low,
                   double high, double old, void* stream);

/* CFG + temperature + top-k + Exponential-race sampler over [B, V] f16 logits (B = 2N with CFG:
 * rows 0..N-1 conditional, N..2N-1 unconditional; B = N without).  For each take n the token is
 * written to out[n * out_stride] (and out[(n + N) * out_stride] with CFG).  The Exponential(1)
 * draws come from Philox4x32-10 keyed by *seed and countered by (index, take, *pos, salt), or
 * from noise [N, V] f32 when noise != NULL.  V <= 8704.
 * Replaces _sample and _guided (app/engine.py:291-305) -- ~25 PyTorch kernels per call. */
int ecd_sample_topk(const void* logits, long ld, int B, int N, float cfg, float temp, int topk,
                    int V, const float* noise, const int64_t* seed, const int64_t* pos, int salt,
                    int64_t* out, long out_stride, void* stream);

/* ecd_sample_topk, then the next depth-decoder pass's input for each sampled token t of take n
 * (rows n and n + N with CFG):
 *  - x rows <- rows[t] from rows [rows_n >= V, D] f16 (row stride rows_ld), row stride x_ld;
 *    rows and x 16-byte aligned, D (at most 3072), rows_ld and x_ld multiples of 8;
 *  - with qkv != NULL, that pass's layer 0 up to its attention output: q | k | v of t from
 *    qkv [qkv_n >= V, (Hq + 2 Hk) * HD] f16 (row stride qkv_ld; q heads, k heads, v heads,
 *    RoPE applied for slot p), k and v into slot p of the caches kc / vc [B, Hk, L, HD], and
 *    the decode attention of each row over slots 0 .. p into o [B, Hq * HD] (row stride o_ld);
 *    Hq / Hk <= 4 and either HD = 128, (1 or 2 rows) * Hk <= 4, p < min(L, 16), or HD = 384
 *    (the arithmetic of ecd_decode_attn's short-cache kernel), (1 or 2 rows) * Hk <= 8,
 *    p < min(L, 8); HD is read only with qkv;
 *  - with ev != NULL, xe rows n (and n + N) <- ev rows n (and n + N), D wide (row strides
 *    ev_ld, xe_ld; 16-byte aligned, multiples of 8): rows that do not depend on the token, such
 *    as the first pass's projected backbone state.
 * A take whose race has no winner (NaN logits) gets zero rows.  With rows[t] =
 * projection(audio embedding of codebook i, token t) and qkv[t] its layer-0 q | k | v at the
 * pass's position, both precomputed by the engine's own kernels, this replaces _guided +
 * projection(_embed_audio(i, ci)) + the decoder's layer-0 rms / q|k|v / RoPE / cache write /
 * attention of one pass (app/engine.py:291-305, 343, 189-199; app/kernels.py:110-153). */
int ecd_sample_topk_next(const void* logits, long ld, int B, int N, float cfg, float temp,
                         int topk, int V, const float* noise, const int64_t* seed,
                         const int64_t* pos, int salt, int64_t* out, long out_stride,
                         const void* rows, long rows_ld, int rows_n, void* x, long x_ld, int D,
                         const void* qkv, long qkv_ld, int qkv_n, void* kc, void* vc, int L,
                         int p, void* o, long o_ld, int Hq, int Hk, int HD, const void* ev,
                         long ev_ld, void* xe, long xe_ld, void* stream);

/* End of one frame of the song loop, on the device (app/engine.py:419-440: the host's
 * tok/pos copies, out[i + 1] = tok[:N] and the EOS scan, moved inside the captured frame).
 *   samples [B, 8] int64 (row stride lds): the frame's tokens; copied into tok [B, 8] (stride
 *   ldt), the next frame's input.  f = pos[0] - P + 1 (every pos row holds the same value);
 *   for 0 <= f <= F rows 0..N-1 are stored in out [F + 1, N, 8] at frame f; for 1 <= f <= F a
 *   take n whose frame holds a token >= eos and whose first_eos[n] is still negative gets
 *   first_eos[n] = f.  Then every pos[b * ldp] (int64 [B]) increases by one.  B <= 64. */
int ecd_frame_advance(const int64_t* samples, long lds, int64_t* tok, long ldt, int64_t* pos,
                      long ldp, int64_t* out, int64_t* first_eos, int B, int N, int P, int F,
                      int64_t eos, void* stream);

/* ---- packed-weight fused GEMVs (the engine's per-layer kernels) ----------------------------
 * Packed layout: [ceil(N/16)] tiles x [K/64] chunks x 1 KB, chunk bytes [16l, 16l+16) holding
 * row 16*tile + (l & 15), bytes 64c + 16(l >> 4) .. +15 (zero rows beyond N).  K % 64 == 0.
 * Every fused variant keeps the numerics of ecd_gemv_i8.  `flags`: bit 0 = dense numerics (the
 * M > 16 path of ecd_gemv_i8), bit 1 = the weights are streamed once (nontemporal loads; leave
 * it clear for weights re-read soon, e.g. the depth decoder's 7 passes, so they stay cached). */

/* Size in bytes of the packed copy of an [N, K] matrix.  No reference counterpart. */
long ecd_packed_bytes(int N, int K);

/* Pack w [N, K] int8 into the tile layout.  interleave = 1 (N even): packed row 2j is row j and
 * row 2j + 1 is row N/2 + j -- the w1 | w3 concatenation of fuse() (app/engine.py:82-86, :112)
 * turned into (a_j, b_j) pairs for the SiLU epilogue.  Offline step like app/convert_final.py. */
int ecd_pack_i8(const void* w, int N, int K, int interleave, void* out, void* stream);

/* int8_mm (app/kernels.py:40-54) on packed weights; nt/kw as in ecd_gemv_i8_tuned. */
int ecd_gemv_i8p(const void* x, long ldx, const void* wp, const void* s, const void* res, long ldr,
                 void* y, long ldy, int M, int N, int K, int flags, int nt, int kw, void* stream);

/* ecd_gemv_i8p with K split over ks workgroups per 16-row tile: each writes fp32 partial sums
 * into the caller's workspace ws [ks, M, N], and a second kernel adds them in split order and
 * applies the scale and residual of ecd_gemv_i8p (same rounding points; the fp32 sum is formed
 * split by split).  For shapes with few output tiles over a long K, where one workgroup per
 * tile leaves most CUs idle (the decoder's w2: N = 1024, K = 8192).  Replaces int8_mm with
 * residual (app/kernels.py:40-54) at app/engine.py:210.  Requires (K / 64) % ks == 0. */
int ecd_gemv_i8p_splitk(const void* x, long ldx, const void* wp, const void* s, const void* res,
                        long ldr, void* y, long ldy, int M, int N, int K, int ks, float* ws,
                        int flags, void* stream);

/* y = int8_mm(rms(x, nw, eps), w, s): rms (app/kernels.py:58-74) fused as the GEMV prologue
 * -- the final norm + head of Stack.decode / _frame_fast (app/engine.py:211, :333, :339). */
int ecd_rms_gemv_i8p(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* y, long ldy, int M, int N, int K, int flags,
                     void* stream);

/* rms -> q|k|v GEMV -> RoPE -> q [M, Hq*HD] and k/v into kc/vc [B, Hk, L, HD] at pos[m]
 * (row m -> batch m / S): app/engine.py:189-192 (krms, b.qkv, _rope_cache) in one kernel.
 * N = (Hq + 2Hk) * HD, HD % 4 == 0; rope [>= L, HD/2, 2] f32.  flags: bit 0 dense numerics,
 * bit 1 streamed weights, bit 2 row output: q is [M, N] and receives q | k | v of row m (RoPE
 * at pos[m] applied to q and k) as its row m; kc and vc are not written (may be NULL). */
int ecd_rms_qkv_rope(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, const float* rope, const int64_t* pos, void* q, void* kc,
                     void* vc, int M, int S, int Hq, int Hk, int L, int HD, int K, int flags,
                     void* stream);

/* rms -> [w1 | w3] GEMV on interleaved packed rows (scales interleaved the same way) ->
 * mm [M, F] = f16(f16(silu(a)) * b): app/engine.py:206-209 (krms, b.w13, _silu_mul). */
int ecd_rms_w13_silu(const void* x, long ldx, const void* nw, float eps, const void* wp,
                     const void* s, void* mm, int M, int F, int K, int flags, void* stream);

/* y = int8_mm(E, w, s) where row m of E is the int8 embedding of tok[m * tok_stride] + cb * vocab
 * (table [trows, K] int8, tscale [trows] f16); with even != NULL (M even) row 2b of E is
 * even[b] (contiguous [M/2, K]) and row 2b + 1 the embedding of tok[b * tok_stride]:
 * projection(_embed_audio(...)) and the pass-0 stack of app/engine.py:336-342. */
int ecd_embed_gemv_i8p(const int64_t* tok, long tok_stride, const void* table, const void* tscale,
                       long trows, int cb, int vocab, const void* even, const void* wp,
                       const void* s, void* y, long ldy, int M, int N, int K, int flags,
                       void* stream);

/* The tail of one decode layer plus the next layer's first steps, as ONE launch (M <= 16 rows):
 *   x1 = xin + int8_mm(o, wo, so)                      app/engine.py:206 (b.o with residual)
 *   mm = fp16(silu(a)) * b, a|b = int8_mm(rms(x1, n2), w13, s13)     :207-208 (krms, b.w13,
 *                                                                      _silu_mul)
 *   xout = x1 + int8_mm(mm, w2, s2)                    :209-210 (b.w2 with residual)
 *   unless wq is NULL (last layer): the next layer's ecd_rms_qkv_rope on xout with n1 / wq / sq
 *   (:189-192): q [M, Hq*HD], k/v into kc/vc [B, Hk, L, HD] at pos (row m -> m / S); and, when
 *   o_next is not NULL, that layer's decode attention (ecd_decode_attn + ecd_attn_combine,
 *   :194-204, scale 1/sqrt(HD)) into o_next [M, Hq * HD] -- for head_dim 128 with 3 or 4 query
 *   heads per kv head, or head_dim 384 with 2 on caches of at most 8 slots
 *   (ecd_layer_tail_supported tells); with several rows per cache (S > 1) the rows of a cache
 *   hold consecutive positions p .. p + S - 1.  M <= 16 rows; the 3072-wide shape takes more
 *   than 8 rows with the head_dim-384 attention or none (the reference decoder's first pass).
 * Same numerics as the per-op entry points up to the fp32 summation order.  wo / w13 / w2 / wq
 * are ecd_pack_i8 copies (w13 interleaved, s13 interleaved the same way); o, xin, x1, mm,
 * xout, o_next 16-byte aligned, row stride D (mm: F).  xout must not alias xin, o, x1 or mm.
 * sync: a 16 KB, 256-byte aligned region, zero before the first call, kept for later calls (the
 * kernel leaves it reusable); calls sharing a sync region must not overlap in time.  err: a
 * 4-byte word made nonzero if a workgroup waited longer than its bound for the others (bit 0,
 * plus one bit per wait that gave up: 2 / 4 / 8 the three gates, 16 the split-W2 parts, 32 / 64
 * the q|k|v hand-off of the VALU / MFMA attention, 128 a new cache slot, 256 the attention
 * merge; results, sync and ws then undefined: zero sync, ws and err before the next call).
 * ws: a 16-byte aligned
 * workspace of ecd_layer_tail_ws_bytes bytes, zero before the first call and kept with its sync
 * region (a launch recognises its split-W2 parts and attention partials by the region's gate
 * count; calls on another sync region must use another ws).  The grid is one workgroup per CU
 * with all workgroups resident.  flags bit 1: nontemporal weight loads; bit 2: no waiting at all
 * (every wait gives up at its first look: tests of the error path); bit 3: nontemporal
 * cache-slot loads for every attention split (without it only splits of more than 32 slots
 * load nontemporal; honoured for head_dim 128 with 3 query heads per kv head, 8 rows).  No
 * reference counterpart as one call: it replaces up to seven reference launches. */
int ecd_layer_tail(const void* o, const void* xin, const void* wo, const void* so,
                   const void* n2, const void* w13, const void* s13, const void* w2,
                   const void* s2, const void* n1, const void* wq, const void* sq,
                   const float* rope, const int64_t* pos, void* q, void* kc, void* vc,
                   void* o_next, void* x1, void* mm, void* xout, void* sync, void* err,
                   void* ws, int M, int D, int F, int S, int Hq, int Hk, int L, int HD,
                   float eps, int flags, void* stream);

/* A stack's first layer up to its attention, as one launch of the ecd_layer_tail kernel without
 * the O projection and the MLP (app/engine.py:189-204 for layer 0): rms(xin, n1) -> q|k|v (wq
 * packed, sq) -> RoPE -> q and the cache slot at pos, and the decode attention into o_next
 * [M, Hq * HD], with q and the new slot handed to the attention as tagged words.  Replaces
 * ecd_rms_qkv_rope + ecd_decode_attn (+ ecd_attn_combine) for the shapes
 * ecd_layer_tail_supported(M, D, F, Hq, Hk, HD, L, 1) accepts (S > 1: the rows of a cache hold
 * consecutive positions, as for ecd_layer_tail); F is
 * the stack's FFN width (the launch shape).  sync, err, ws and flags as for ecd_layer_tail,
 * sync, err and ws shared with the stack's ecd_layer_tail calls (the launch moves the gate count
 * on by one).  No reference counterpart as one call. */
int ecd_layer_head(const void* xin, const void* n1, const void* wq, const void* sq,
                   const float* rope, const int64_t* pos, void* q, void* kc, void* vc,
                   void* o_next, void* sync, void* err, void* ws, int M, int D, int F, int S,
                   int Hq, int Hk, int L, int HD, float eps, int flags, void* stream);

/* ECD_OK when ecd_layer_tail accepts these shapes on the current device (M rows, model width
 * D, FFN width F, heads, L cache slots; attention != 0: with the next layer's attention in the
 * launch), ECD_ENOTSUP otherwise.  No reference counterpart. */
int ecd_layer_tail_supported(int M, int D, int F, int Hq, int Hk, int HD, int L, int attention);

/* Bytes of the ecd_layer_tail workspace for these shapes on the current device.  No reference
 * counterpart. */
long ecd_layer_tail_ws_bytes(int D, int Hq, int Hk, int HD);

/* Layer stacks: nl consecutive ecd_layer_tail calls of one decode step as ONE launch (the loop
 * over layers of app/engine.py:186-210 from layer 0's O projection on).  Layer l's attention
 * output (its o_next) is layer l + 1's o and its xout is layer l + 1's xin; between layers the
 * launch's workgroups meet at one more gate instead of a launch boundary, and the next layer's
 * weights stream during it.  A layer is described by the pointers of ecd_layer_tail that change
 * from layer to layer, in this order: */
typedef struct ecd_layer_rec {
  const void* wo;   /* packed W_O, scales, post-attention norm weights */
  const void* so;
  const void* n2;
  const void* w13;  /* packed row-interleaved w1 | w3, scales; packed w2, scales */
  const void* s13;
  const void* w2;
  const void* s2;
  const void* n1;   /* the next layer's input norm, packed q|k|v and scales, K/V caches; */
  const void* wq;   /* NULL (with n1, sq, kc, vc, o_next) only for the stack's last layer */
  const void* sq;
  void* kc;
  void* vc;
  void* x1;         /* this layer's outputs: [M, D], [M, F], [M, D]; o_next [M, Hq * HD] */
  void* mm;
  void* xout;
  void* o_next;
  void* y;          /* the last layer of a 1024-wide stack only, or NULL: it ends in a codebook */
} ecd_layer_rec;    /* head, y [M, yn] (row stride yld) = fp16(s * (w rms(xout, n1))) with n1, */
                    /* wq, sq the head's norm, packed weights and scales (no kc, vc, o_next) */
#define ECD_STACK_MAX 64 /* layers per stack */

/* Checks nl records on the host and copies them to plan (device memory of
 * ecd_layer_stack_plan_bytes(nl) bytes, 16-byte aligned), synchronously on stream.  Every layer
 * but the last must run the next layer's q|k|v and attention; the outputs x1, mm, xout, o_next
 * and y of all layers must be pairwise disjoint (within one launch no buffer is written twice,
 * so no XCD's L2 can hold an older copy of a line it reads); yld: the row stride of y (0: no
 * head).  No reference counterpart. */
int ecd_layer_stack_plan(const void* layers, int nl, int M, int D, int F, int Hq, int Hk,
                         int HD, int yld, void* plan, void* stream);
long ecd_layer_stack_plan_bytes(int nl);

/* ECD_OK when ecd_layer_stack runs nl layers of these shapes with these flags (bit 1 streamed
 * weights, bit 3 nontemporal cache-slot loads) on the current device: the backbone (3072 wide,
 * 24q / 8kv, head_dim 128, streamed weights, up to 8 rows, a multiple of 7 layers: 7 per
 * launch) and the two depth decoders (3072 wide with head_dim 384, 1024 wide with head_dim 128;
 * caches of at most 8 slots; up to 16 rows; weights not streamed; all layers in one launch).
 * No reference counterpart. */
int ecd_layer_stack_supported(int nl, int M, int D, int F, int Hq, int Hk, int HD, int L,
                              int flags);

/* Layers per kernel launch of an ecd_layer_stack call with these arguments (nl / that many
 * launches), or ECD_ENOTSUP.  No reference counterpart. */
int ecd_layer_stack_layers_per_launch(int nl, int M, int D, int F, int Hq, int Hk, int HD, int L,
                                      int flags);

/* One launch for the nl layers of plan (written by ecd_layer_stack_plan): layer 0 starts from o
 * and xin [M, D]; the result is the last layer's xout (and, with a head record, its logits y:
 * yn columns, row stride yld; yn = 0 without).  rope, pos, q, sync, err, ws, the shapes, eps
 * and flags as for ecd_layer_tail, shared by every layer (err bit 512: an o gate gave up); q
 * receives the last q|k|v step's queries.  Replaces nl ecd_layer_tail calls (and the head's
 * ecd_rms_gemv_i8p); no reference counterpart as one call. */
int ecd_layer_stack(const void* plan, int nl, const void* o, const void* xin, const float* rope,
                    const int64_t* pos, void* q, void* sync, void* err, void* ws, int M, int D,
                    int F, int S, int Hq, int Hk, int L, int HD, int yn, int yld, float eps,
                    int flags, void* stream);

/* Prompt-pass GEMM (many rows) on packed weights: y = fp16(x @ fp16(q * s)^T) (+ res as an
 * fp16 add) -- the dense numerics of int8_mm for M > 16 (app/kernels.py:46-49), used by the
 * prompt pass (app/engine.py:123-153, 174-178).  MFMA-tiled 128 x 128 per workgroup.
 *   x [M, K] fp16 (row stride ldx, 16-byte aligned, K % 64 == 0); wp = ecd_pack_i8(w);
 *   s [N] fp16; res [M, N] (row stride ldr) or NULL; y [M, N] (row stride ldy).
 *   ECD_ENOTSUP when M * ldx * 2 bytes reach 2 GiB (32-bit per-lane load offsets). */
int ecd_gemm_i8p(const void* x, long ldx, const void* wp, const void* s, const void* res,
                 long ldr, void* y, long ldy, int M, int N, int K, void* stream);

/* The same GEMM on row-interleaved w1|w3 (ecd_pack_i8 with interleave) with the SiLU * mul
 * epilogue: mm[m, j] = fp16(fp16(silu(a_j)) * b_j), a/b the GEMM outputs of rows 2j / 2j + 1
 * (app/engine.py:152-153, app/kernels.py:171-180).  mm [M, F] (row stride ldm). */
int ecd_gemm_i8p_silu(const void* x, long ldx, const void* wp, const void* s, void* mm,
                      long ldm, int M, int F, int K, void* stream);

/* The same GEMM on the packed q | k | v projection (N = (Hq + 2 Hk) * HD) with the RoPE +
 * KV-cache write of app/kernels.py:78-107 in its epilogue (replaces int8_mm + _rope_cache in
 * the prompt pass, app/engine.py:123-153): y = fp16(x @ fp16(q * s)^T) as ecd_gemm_i8p, then
 * row m (batch item m / S, position pos[m]) rotates the interleaved pairs of its q and k heads
 * by rope[p] (fp32, rounded to fp16; p = pos[m] clamped into [0, L)) and writes q [M, Hq * HD],
 * and k, v into kc / vc [B, Hk, L, HD] at slot pos[m] when 0 <= pos[m] < L -- the outputs of
 * ecd_rope_kv_write on the GEMM's output.  HD % 4 == 0; rope 16-byte aligned; q, kc, vc 8-byte
 * aligned. */
int ecd_gemm_i8p_rope(const void* x, long ldx, const void* wp, const void* s, const float* rope,
                      const int64_t* pos, void* q, void* kc, void* vc, int M, int S, int Hq,
                      int Hk, int L, int HD, int K, void* stream);

/* fp16-weight GEMM of the codec's flow-matching estimator (the dense nn.Linear / Conv1d-as-GEMM
 * layers of app/heartcodec/models/transformer.py; torch's F.linear numerics: fp32 accumulation,
 * fp32 bias, one fp16 rounding).  Weights are packed once with ecd_pack_f16 into lane-ordered
 * 16 x 64 tiles of 2 KB (ecd_packed_bytes_f16 bytes; rows beyond N zero).
 *   ecd_gemm_f16p:      y = fp16(x @ w^T + bias); if alpha != 1, y = fp16(y * alpha); then
 *                       y += res (fp16 add).  bias [N] fp32 or NULL, res [M, N] or NULL.
 *   ecd_gemm_f16p_silu: w packed with interleave (gate | up), mm[m, j] =
 *                       fp16(fp16(silu(g)) * u) with g, u the fp16 GEMM outputs (LlamaMLP,
 *                       transformer.py:181-184).
 * x [M, K] fp16 (row stride ldx, 16-byte aligned, K % 64 == 0); ECD_ENOTSUP when M * ldx * 2
 * bytes reach 2 GiB. */
long ecd_packed_bytes_f16(int N, int K);
int ecd_pack_f16(const void* w, int N, int K, int interleave, void* out, void* stream);
int ecd_gemm_f16p(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                  const void* res, long ldr, void* y, long ldy, int M, int N, int K, void* stream);
int ecd_gemm_f16p_silu(const void* x, long ldx, const void* wp, void* mm, long ldm, int M, int F,
                       int K, void* stream);

/* The same GEMM with nn.PReLU (one slope) after the bias and rounding, then the optional fp16
 * residual: y = fp16(acc + bias); y < 0 -> fp16(slope * y); y = fp16(y + res).  The conv ->
 * PReLU (-> + x) steps of the codec's waveform decoder (app/heartcodec/models/sq_codec.py:
 * 149-168), with the convolution as a GEMM over tap columns (ecd_codec_cols_taps). */
int ecd_gemm_f16p_prelu(const void* x, long ldx, const void* wp, const float* bias, float slope,
                        const void* res, long ldr, void* y, long ldy, int M, int N, int K,
                        void* stream);

/* A convolution as this GEMM over implicit tap columns, time-major rows m = b*T + t (M % T == 0):
 * with k taps, x holds each sequence after xpad zero rows and K = k*C, the columns of row m being
 * the source rows at offsets[j] from it; k = 0: x is plain [M, K].  rep = 1: source sequences of T
 * rows (row b*(T + xpad) + xpad + t); rep = 2: the source is upsampled 2x by row repeat (nearest),
 * so it holds T/2 rows per sequence and output step t, tap o reads source row (t + o) >> 1 (T even).
 * Every source row read stays within the zero padding (|offsets| <= xpad, halved with rep 2); the
 * caller also leaves that many zero rows after the last sequence.  With ypad >= 0, y and res rows
 * are b*(T + ypad) + ypad + t, else plain.  epi 0 (store, alpha the scale) or 2 (PReLU, alpha the
 * slope).  The causal and dilated Conv1d, ConvTranspose1d and the PostProcessor's upsample + conv
 * of the codec's waveform decoder (sq_codec.py:32-287) without materialised columns. */
int ecd_gemm_f16p_conv(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                       const void* res, long ldr, void* y, long ldy, int M, int N, int K, int T,
                       int xpad, int ypad, const int* offsets, int k, int rep, int epi,
                       void* stream);

/* ecd_gemm_f16p_conv with an explicit block tile (cfg as in ecd_gemm_f16p_tuned; 0 = the
 * library's choice).  Replaces nothing in the reference: the launch-shape knob of the waveform
 * decoder's convolutions, for sweeps and for the tests that hold every tile to the same bits. */
int ecd_gemm_f16p_conv_tuned(const void* x, long ldx, const void* wp, const float* bias,
                             float alpha, const void* res, long ldr, void* y, long ldy, int M,
                             int N, int K, int T, int xpad, int ypad, const int* offsets, int k,
                             int rep, int epi, int cfg, void* stream);

/* ecd_gemm_f16p (epi 0), ecd_gemm_f16p_silu (epi 1, N = 2F, bias/res NULL, alpha 1) or
 * ecd_gemm_f16p_prelu (epi 2, alpha = the slope) with an
 * explicit block tile (cfg 1..16: 128x128, 256x128, 128x256, 128x64, 64x128, 64x256, 64x64 or 128x96 features x rows,
 * 2 to 4 LDS stages; 0 = the library's choice).  Replaces nothing in the reference: the launch-shape knob
 * of the codec GEMMs, for sweeps. */
int ecd_gemm_f16p_tuned(const void* x, long ldx, const void* wp, const float* bias, float alpha,
                        const void* res, long ldr, void* y, long ldy, int M, int N, int K,
                        int epi, int cfg, void* stream);

/* Causal attention of the prompt pass on MFMA: row r = b * S + s of q [B * S, Hq * HD] attends
 * cache slots [0, pos[r]] of kc, vc [B, Hk, L, HD] (the prompt's K/V already written), with the
 * decode kernel's numerics (fp32 scores, running max, fp16 probabilities into P.V, fp32 sums).
 * Replaces the causal scaled_dot_product_attention of the prompt pass (app/engine.py:123-153,
 * :174-178).  o [B * S, Hq * HD].  HD in {64, 128}; Hq / Hk in {1, 2, 3, 4}; scale > 0; q, kc,
 * vc 16-byte and o 8-byte aligned.  With pos[r] = S - 1 for every row and L = S it is non-causal attention over
 * the sequence (the codec estimator, app/heartcodec/models/transformer.py:117-125). */
int ecd_prefill_attn(const void* q, const void* kc, const void* vc, const int64_t* pos, void* o,
                     int B, int S, int Hq, int Hk, int L, int HD, float scale, void* stream);

/* ---- codec flow-matching estimator glue (app/heartcodec/models/transformer.py,
 * app/heartcodec/models/flow_matching.py).  All tensors fp16 unless stated, 16-byte aligned,
 * rounded to fp16 at the points where the reference's eager fp16 ops round. */

/* RoPE table tab [T, HD/2] of (cos, sin) fp16 pairs, computed in fp16 like
 * RotaryEmbedding.get_sin_cos (transformer.py:28-42, base 10000). */
int ecd_codec_rope_table(void* tab, int T, int HD, void* stream);

/* Interleaved RoPE on the q and k heads of qkv [B*T, ldq] (q | k | v, H*HD columns each) ->
 * q [B*T, H*HD], k and v [B, H, T, HD] (apply_rope_vec, transformer.py:108-122). HD % 8 == 0. */
int ecd_codec_rope_heads(const void* qkv, long ldq, const void* tab, void* q, void* k, void* v,
                         int B, int T, int H, int HD, void* stream);

/* The q | k | v projection with the RoPE above fused into the GEMM epilogue:
 * qkv = fp16(x @ w^T + bias) (ecd_gemm_f16p, w packed [3 H HD, K]), then q, k, v as
 * ecd_codec_rope_heads writes them (same rounding, bit for bit), without the qkv buffer.
 * x [M, K] (M = B T rows b T + t), tab as above, q [M, H HD], k and v [B, H, T, HD], 8-byte
 * aligned; HD % 4 == 0.  Replaces to_q / to_k / to_v + apply_rope_vec (transformer.py:108-122,
 * 219-226) in one launch. */
int ecd_gemm_f16p_rope(const void* x, long ldx, const void* wp, const float* bias,
                       const void* tab, void* q, void* k, void* v, int M, int T, int H, int HD,
                       int K, void* stream);

/* Row r of x [R, D] (batch r / T): with h, x = fp16(x + fp16(fp16(g_tab + g_tm[b]) * h)) in
 * place (the gated residual, transformer.py:241-248); then norm 0 = RMSNorm with weight w
 * (:9-18), norm 1 = LayerNorm without affine (:333-334), and
 * y = fp16(fp16(n * fp16(1 + scale)) + shift) with shift = fp16(sh_tab + sh_tm[b]),
 * scale = fp16(sc_tab + sc_tm[b]) (:234-239, :366-370).  g_tm of batch b starts at b * g_ld,
 * sh_tm and sc_tm at b * tm_ld (0: shared).  D % 8 == 0, D <= 4096. */
int ecd_codec_norm_mod(void* x, const void* h, const void* g_tab, const void* g_tm, long g_ld,
                       const void* w, const void* sh_tab, const void* sh_tm, const void* sc_tab,
                       const void* sc_tm, long tm_ld, void* y, int R, int T, int D, int norm,
                       float eps, void* stream);

/* Columns of nn.Conv1d(k = 3, padding = 1) (ProjectLayer, transformer.py:258-272) over the
 * channel concatenation of up to 4 segments: out [B*T, 3*C], out[b*T + t, j*C + c] =
 * in[b, t + j - 1, c] (zero outside [0, T)); segment i gives seg_w[i] channels from
 * seg_ptr[i] + ((b % seg_bmod[i]) * (T / r) + s / r) * seg_ld[i], r = seg_rep[i] (1 if
 * seg_rep is NULL; 2 reads a half-rate source as its nearest 2x upsampling,
 * flow_matching.py:106-108), for b >= seg_bzero[i], zeros below (solve_euler's input,
 * flow_matching.py:183-193; torch.cat of transformer.py:372). */
int ecd_codec_cols3(const void* const* seg_ptr, const long* seg_ld, const int* seg_w,
                    const int* seg_bmod, const int* seg_bzero, const int* seg_rep, int nseg,
                    void* out, int B, int T, void* stream);

/* Code embedding: out [B*Tc, Wp] fp16, out[b*Tc + t, d] = fp16(sum_q books[q, codes[b, q, t], d])
 * for d < Dc, zero for Dc <= d < Wp (ResidualVQ.get_codes_from_indices and the sum over
 * quantizers, flow_matching.py:98-99); books [Q, V, Dc] fp16; codes int64 at
 * codes[b*cb + q*cq + t].  clamp 0: codes -1 or outside [0, V) contribute nothing; clamp 1:
 * codes are clamped to [0, V - 1] first (app/codec_lite.py:71).  Dc, Wp % 8 == 0. */
int ecd_codec_vq_embed(const int64_t* codes, long cb, long cq, const void* books, void* out,
                       int B, int Q, int Tc, int V, int Dc, int Wp, int clamp, void* stream);

/* ---- codec waveform decoder (app/heartcodec/models/sq_codec.py ScalarModel.decode), time-major
 * activations [B, T, C]. */

/* Tap columns of a 1-D convolution for global rows row0 .. row0 + nrows - 1 (row = b*T + t):
 * out[row - row0, j*C + c] = src[b, (t + offsets[j]) / rep, c] for 0 <= t + offsets[j] < T,
 * else 0 (src [B, spad + T / rep, C], row stride ld, spad rows before each sequence; k <= 8 taps,
 * rep 1 or 2).  Causal Conv1d: offsets (j - k + 1) * dilation (sq_codec.py:32-73); causal
 * ConvTranspose1d with kernel 2s, stride s (sq_codec.py:76-117): offsets {0, -1}, the GEMM's
 * [T, s*Cout] output being the upsampled [T*s, Cout]; rep 2: PostProcessor's 2x repeat
 * (sq_codec.py:140-146).  C % 8 == 0. */
int ecd_codec_cols_taps(const void* src, long ld, const int* offsets, int k, void* out, int B,
                        int T, int C, int rep, int spad, long row0, long nrows, void* stream);

/* Weight normalisation (torch.nn.utils.parametrizations.weight_norm, dim 0): w[r, :] =
 * fp16(v[r, :] * (g[r] / |v[r, :]|)), fp32 norm, rows of n contiguous values. */
int ecd_codec_weight_norm(const void* v, const void* g, void* w, int rows, int n, void* stream);

/* One window's latent lat [T, S*Cl] -> out [S, T, Cl], out[s, t, c] = round(9 x) / 9 in fp16
 * (modeling_heartcodec.py:176-183, ScalarModel.decode's round_func9, sq_codec.py:368-372). */
int ecd_codec_latent_split(const void* lat, void* out, int T, int S, int Cl, void* stream);

/* Timestep sinusoid out [n, 512] fp16 from t [n] fp32 (PixArtAlphaCombinedFlowEmbeddings.
 * timestep_embedding, transformer.py:408-426). */
int ecd_codec_timestep(const float* t, void* out, int n, void* stream);

/* y = fp16(silu(x)) over n elements (nn.SiLU, transformer.py:435, 451). */
int ecd_codec_silu(const void* x, void* y, long n, void* stream);

/* One Euler step on x [B, T, C]: with cfg 1, dphi [2B, T, C] (unconditional half first) is
 * combined with guidance g; with cfg 0, dphi [B, T, C] is the velocity (dphi NULL: no update).
 * Then on rows t < L: mode 0 the in-context blend at time tb for the next estimator call,
 * mode 1 the in-context latents (FlowMatching.solve_euler, flow_matching.py:179-203, and
 * :156-158).  C % 8 == 0. */
int ecd_codec_euler(void* x, const void* noise, const void* ic, const void* dphi, int cfg, int B,
                    int T, int C, int L, float dt, float g, float tb, int mode, void* stream);

/* Plain device-to-device byte copy (nbytes and both pointers 16-byte aligned).  No reference
 * counterpart: a kernel of known HBM traffic used to calibrate hardware byte counters. */
int ecd_copy_bytes(const void* src, void* dst, long nbytes, void* stream);

/* Library version string (static storage). */
const char* ecd_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ECDECODE_H */
