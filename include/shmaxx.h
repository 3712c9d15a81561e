/* C ABI of libshmaxx.so: the MI355X (gfx950) kernels of the strix-halo-maxx hot path.
 *
 * Conventions (same style as the reference's launchers, moondream/gpu/hip/i8gemm.hip:478-595, attn.hip:433-462):
 *  - plain C types only: hipStream_t, raw device pointers, element counts/strides (in elements, not bytes);
 *  - bf16 tensors are passed as uint16_t* bit patterns, fp32 as float*;
 *  - every entry point launches asynchronously on the given stream, never allocates, frees or synchronises, and
 *    returns 0 or a negative status:
 *      -1 unknown config / head dim / mode   -2 unsupported shape or stride   -3 workspace too small
 *      -4 pointer alignment / layout         -5 HIP launch failed             -6 required pointer is null
 *  - shapes are validated on the host before any launch (the *_check functions run that validation alone);
 *  - every entry point is HIP-graph capturable (no host reads of device data, no memsets).
 */
#ifndef SHMAXX_H
#define SHMAXX_H
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ============================================================================================ GEMM (MFMA)
 * C[M,N] = epi(A[M,K] . W[N,K]^T + bias[N]); the k loop runs to Kw (multiple of 64, >= K), W must be zero in
 * columns [K, Kw). act: 0 none, 1 GELU-tanh, 2 GELU-erf (applied to the bf16-rounded linear output; with
 * act_ncols > 0 only on output columns < act_ncols), 3 gated GELU-tanh on interleaved (gate, up) weight rows
 * (output width N / 2). Then "+ R" (R row = m % r_rows when r_rows > 0, else m), each step rounded to bf16.
 * cfg < 0: the library's tile pick; splits > 1 needs ws (fp32) and cnt (ints, zero before first use, left zero).
 * Requirements: K % 8 == 0, lda/ldw % 8 == 0, A/W 16-byte aligned, N % 4 == 0, bias 16-byte aligned.
 * Replaces: bf16gemm_launch (moondream/gpu/hip/i8gemm.hip:534-552, bound in moondream/gpu/hgemm.py:28) with its
 * `gelu` flag; the residual the reference adds outside the GEMM (md2fast.py:64-67); the gated-MLP epilogue of the
 * TRecViT ffw_up (tapnext/npu/NOTES.md:36, pack8.py:96-102 interleave_gated). */
int mx_gemm_bf16(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                 const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int K,
                 int Kw, int act, int act_ncols, float* ws, long ws_elems, int* cnt, long n_cnt);
/* Host-only validation of an mx_gemm_bf16 call. Replaces the shape checks at i8gemm.hip:535, :557-561. */
int mx_gemm_check(int cfg, int splits, const void* A, long lda, const void* W, long ldw, const void* bias,
                  const void* R, long ldr, const void* C, long ldc, int M, int N, int K, int Kw, int act,
                  const void* ws, long ws_elems, const void* cnt, long n_cnt);
/* Default (cfg * 16 + splits) for (M, N, Kw). Replaces pick_cfg's FIXED table (moondream/gpu/hgemm.py:47-51). */
int mx_gemm_pick(int M, int N, int Kw);
/* Number of tile configs / the (BM, BN) tile of one. Replaces bf16gemm_ncfg (i8gemm.hip:553). */
int mx_gemm_ncfg(void);
int mx_gemm_cfg_tile(int cfg, int* bm, int* bn);
/* Kernel kind of a tile config: 0 = LDS-shared tile (split-K capable), 1 = wave-split K (splits must be 1 in
 * mx_gemm_bf16; mx_gemm_bf16_partial splits K over workgroups), or MX_EBADCFG. No counterpart in the reference (its
 * configs are all one kind). */
int mx_gemm_cfg_kind(int cfg);
/* Raw split-K partials for a 4-wave cfg (either kind) or a two-k-group 8-wave cfg (19-22; the other 8-wave cfgs return
 * MX_EBADCFG): P[s][m][n] = sum over split
 * s's k-steps of A[m,k] W[n,k] (fp32; row stride ldp, split stride p_split), no bias / activation / residual; the
 * consumer adds the splits in order
 * (mx_residual_layernorm). No counterpart in the reference (no split-K there): it replaces the GEMM half of the
 * residual Linears x + proj(a) and x + fc2(f) (moondream/gpu/md2fast.py:152-157). */
int mx_gemm_bf16_partial(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                         float* P, long ldp, long p_split, int M, int N, int K, int Kw);
/* C = epi(sum over s < nsplit of P[s] + bias), mx_gemm_bf16's epilogue (act 0-3, act_ncols, + R with r_rows) on raw
 * partials of mx_gemm_bf16_partial, splits added in order; one split equals mx_gemm_bf16 bit for bit. With the
 * partial GEMM it is the fence-free split-K of the small-M GEMMs (prompt and query rows): it stands for the
 * reference's small-M split-K path (i8gemm_small_launch, moondream/gpu/hip/i8gemm.hip:555-592, chosen at
 * moondream/gpu/hgemm.py:120-122). N % 4 == 0, ldp % 4 == 0, P 16-byte and C 8-byte aligned (4-byte for act 3). */
int mx_gemm_reduce(hipStream_t st, const float* P, int nsplit, long p_split, long ldp, const float* bias,
                   const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int act,
                   int act_ncols);
/* Residual Linear and the LayerNorm that reads it, in one launch: X = bf16(bf16(A W^T + bias) + R) and Y =
 * LayerNorm(X; gamma, beta, eps), the roundings of mx_gemm_bf16_partial + mx_residual_layernorm. Replaces the
 * block's lin_res(proj) + ln2 and lin_res(fc2) + the next block's ln1 (moondream/gpu/md2fast.py:153-157, the post-LN
 * at :158 for the last block), and TRecViT's `x2 = out_proj(a) + x1; ln_2(x2)` (tapnext/npu/step8.py:484-487). The
 * 64 x 64 output tiles of a row block exchange their rows' sums and centred square sums through stats (>=
 * mx_gemm_res_ln_stats_words(M, N) 64-bit words) and wait for each other, so the whole grid must be resident: N % 64
 * == 0, N <= 4096 and ((M + 63) / 64) * (N / 64) <= the device's CU count, else MX_ESHAPE. sync (>=
 * mx_gemm_res_ln_sync_words(M) 32-bit words) and stats are zeroed once by the caller and then kept ready by the
 * kernel; calls that share them must be ordered on one stream and have the same N (any M): where a row block's words
 * sit depends on N / 64, so a call of another N could meet old words carrying the epoch it expects and accept stale
 * statistics. Give each N its own stats / sync. sync[0] != 0 after a call: a wait timed out and the results are
 * undefined (zero both before the next call). The statistics combine per-tile sums in fp32 in another order than
 * mx_residual_layernorm's row sums (Y within a bf16 rounding of it; X identical for the same k-loop). */
int mx_gemm_bf16_res_ln(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
                        const uint16_t* R, long ldr, uint16_t* X, long ldx, const uint16_t* gamma,
                        const uint16_t* beta, uint16_t* Y, long ldy, int M, int N, int K, int Kw, float eps,
                        uint64_t* stats, long stats_words, uint32_t* sync, long sync_words);
/* The same launch with the TRecViT RMSNorm in place of the LayerNorm: X as above, Y = bf16(bf16(X rstd) sc1) with
 * rstd = bf16(1 / sqrt(bf16(bf16(sum bf16(X^2) / N) + eps))), sc1 = bf16(scale + 1), the roundings of
 * mx_residual_rmsnorm. Replaces TRecViT's `x1 = linear_out(z) + x; channel_pre_norm(x1)` (tapnext/npu/step8.py:480-482;
 * RMSNorm numerics tapnext/npu/pack8.py:222-229) where the grid fits (one frame: 20 x 12 tiles). The tiles exchange
 * their rows' sums of bf16(X^2) (another fp32 summation order than the row kernel's, before the bf16 rounding of the
 * mean square). Same shape rules, stats / sync words and error word as mx_gemm_bf16_res_ln; calls of either form
 * with the same N may share them when ordered on one stream. */
int mx_gemm_bf16_res_rms(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
                         const uint16_t* R, long ldr, uint16_t* X, long ldx, const uint16_t* sc1, uint16_t* Y,
                         long ldy, int M, int N, int K, int Kw, float eps, uint64_t* stats, long stats_words,
                         uint32_t* sync, long sync_words);
long mx_gemm_res_ln_stats_words(int M, int N);
long mx_gemm_res_ln_sync_words(int M);

/* mx_gemm_bf16 without a caller workspace: in-kernel split-K (splits > 1, or a split pick when cfg < 0) uses a fixed
 * device array of the library (mx_gemm_noalloc_max_ws() fp32 partial elements, 16 MiB, plus 65,536 tile counters)
 * instead of ws / cnt; a call needing more returns -3 before launching. It allocates nothing (no hipMalloc, no torch
 * allocation) and clears the counters it uses with a kernel, so it can be captured into a HIP graph. Each GPU holds
 * its own copy of the array for the life of the process, and every such call on a GPU shares it: calls that overlap
 * on one GPU (different streams) race. No counterpart in the reference: it is for callers that cannot allocate
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int mx_gemm_bf16_noalloc(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                         const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M,
                         int N, int K, int Kw, int act, int act_ncols);
long mx_gemm_noalloc_max_ws(void);

/* ============================================================================================ W8A8 (int8 MFMA)
 * Per-token int8 quantisation of bf16 activations: s[m] = max(max_k |x[m,k]|, 1e-5) / 127 and
 * q[m,k] = trunc(x / s + 0.5 sign) (round half away from zero), fp32 math with IEEE division. K % 8 == 0; strides in
 * elements (ldx bf16, ldq int8 bytes; multiples of 8). Replaces the reference's _quant_rows / quant_rows
 * (moondream/gpu/tgemm.py:81-91, hgemm.py:10-16). */
int mx_quant_rows_i8(hipStream_t st, const uint16_t* x, long ldx, int8_t* q, long ldq, float* s, int M, int K);
/* Per-output-channel int8 quantisation of a bf16 weight: s[n] = max(max_k |w[n,k]|, 1e-8) / 127 and
 * q[n,k] = clamp(round-half-even(w / s), -127, 127), fp32 with IEEE division (columns past K of q untouched).
 * Replaces the weight quantisation of HI8Lin.__init__ (moondream/gpu/hgemm.py:101-106). */
int mx_quant_weight_i8(hipStream_t st, const uint16_t* w, long ldw, int8_t* q, long ldq, float* s, int N, int K);
/* W8A8 GEMM: C = bf16(act(((float)(A W^T) * sa[m]) * sw[n] + bias[n])) [then + R, rounded again]: A (M, K) and
 * W (N, Kw) int8, row strides lda / ldw in BYTES (multiples of 16), K % 16 == 0, Kw % 128 == 0, W zero in columns
 * [K, Kw); sa / sw fp32 per-row / per-column scales; act 0 none, 1 GELU-tanh, 2 GELU-erf, applied to the fp32 value
 * before the one bf16 rounding. With P (int32, row stride ldp elements) the raw accumulators are written instead and
 * sa / sw / bias / R / C are ignored (cfg must then have a partial-sum mode). cfg: a kind-0 tile config
 * (mx_gemm_cfg_kind == 0). Replaces i8gemm_launch (moondream/gpu/hip/i8gemm.hip:480) with its epilogue
 * (i8gemm.hip:181-197); the fused residual stands for the reference's separate bf16 add (md2fast.py:55-67). */
int mx_gemm_i8(hipStream_t st, int cfg, const int8_t* A, long lda, const int8_t* W, long ldw, const float* sa,
               const float* sw, const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M,
               int N, int K, int Kw, int act, int32_t* P, long ldp);
/* W8A8 split-K for the small-M GEMMs: raw int32 partials of `splits` contiguous k ranges (P[s][m][n], row stride ldp,
 * split stride p_split; kind-0 configs with a partial-sum mode), then mx_gemm_i8_reduce: the exact int32 sum of
 * the partials through mx_gemm_i8's epilogue, so the pair equals mx_gemm_i8 bit for bit for any split count. Stands
 * for the reference's small-M int8 split-K (i8gemm_small_launch + its reduce, moondream/gpu/hip/i8gemm.hip:389-443,
 * :555-592). */
int mx_gemm_i8_partial(hipStream_t st, int cfg, int splits, const int8_t* A, long lda, const int8_t* W, long ldw,
                       int32_t* P, long ldp, long p_split, int M, int N, int K, int Kw);
int mx_gemm_i8_reduce(hipStream_t st, const int32_t* P, int nsplit, long p_split, long ldp, const float* sa,
                      const float* sw, const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C,
                      long ldc, int M, int N, int act);
/* Split-K workspace a (cfg, splits) call needs: fp32 elements / tile counters. Replaces the fixed-size
 * workspace() of moondream/gpu/hgemm.py:78-83. */
long mx_gemm_ws_elems(int cfg, int splits, int M, int N);
long mx_gemm_ws_counters(int cfg, int splits, int M, int N);

/* ============================================================================================ attention
 * O[b, i, h*D + d] = softmax(scale * Q K^T) V over visible keys; key j visible to query i iff j < Tk and
 * (j < causal_from || j <= qpos0 + i). D in {64, 72}. Q/K/V/O addressed as base + b*s_b + h*s_h + t*s_t + d.
 * Replaces: attn_fwd2 + vtranspose (moondream/gpu/hip/attn.hip:442-451, :275-288; bound in moondream/gpu/hattn.py:11-14),
 * which are mask-free and batch 1; the masked prompt prefill (md2fast.py:132-136, :185) and the TRecViT attention
 * (tapnext/npu/step8.py:484-486) used torch SDPA there. */
int mx_sdpa(hipStream_t st, const uint16_t* Q, long sq_b, long sq_h, long sq_t, const uint16_t* K, long sk_b,
            long sk_h, long sk_t, const uint16_t* V, long sv_b, long sv_h, long sv_t, uint16_t* O, long so_b, long so_h,
            long so_t, int B, int H, int Tq, int Tk, int D, float scale, int qpos0, int causal_from);
int mx_sdpa_check(const void* Q, long sq_t, const void* K, long sk_t, const void* V, long sv_t, const void* O,
                  long so_t, int B, int H, int Tq, int Tk, int D);
/* The tiling mx_sdpa picks for (B, H, Tq, D): t[0..3] = query waves, key waves, keys per staged block, ring stages
 * (the kernel is attn_fwd_kernel<D, t0, t1, t2, t3>). The reference picks its tile from a fixed table by head dim
 * (moondream/gpu/hattn.py:21); this one also looks at the grid size. */
void mx_sdpa_tiling(int B, int H, int Tq, int D, int* t);

/* ============================================================================================ norms
 * LayerNorm over rows of D (fp32 statistics, one rounding). Replaces F.layer_norm in _ln (md2fast.py:43-44) and the
 * TRecViT ln_1 / ln_2 / encoder_norm (numerics restated at tapnext/npu/pack8.py:232-238). */
int mx_layernorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* gamma, const uint16_t* beta, uint16_t* Y,
                 long ldy, int rows, int D, float eps);
/* x = bf16(bf16(sum_s P[s] + bias) + R) -> Xo, then y = LayerNorm(x) -> Y (skipped when gamma is null): the
 * epilogue of a split-K residual Linear fused with the LayerNorm that reads its output. Replaces the residual add +
 * next _ln of the vision block loop (moondream/gpu/md2fast.py:152-157, :43-44); bias fp32 or null. */
int mx_residual_layernorm(hipStream_t st, const float* P, int nsplit, long p_split, long ldp, const float* bias,
                          const uint16_t* R, long ldr, uint16_t* Xo, long ldxo, const uint16_t* gamma,
                          const uint16_t* beta, uint16_t* Y, long ldy, int rows, int D, float eps);
/* The same reduction with the TRecViT RMSNorm of x -> Y (sc1 = bf16(scale + 1), required): the residual Linear of a
 * TRecViT block fused with the RMSNorm that reads its output, i.e. `res = linear_out(z) + x; channel_pre_norm(res)`
 * and `x3 = mlp3(...) + x2; next block's temporal_pre_norm(x3)` (tapnext/npu/step8.py:470-488; the RMSNorm numerics of
 * tapnext/npu/pack8.py:222-229). At most 4 splits, D <= 2048. */
int mx_residual_rmsnorm(hipStream_t st, const float* P, int nsplit, long p_split, long ldp, const float* bias,
                        const uint16_t* R, long ldr, uint16_t* Xo, long ldxo, const uint16_t* sc1, uint16_t* Y,
                        long ldy, int rows, int D, float eps);
/* TRecViT RMSNorm with torch's bf16 rounding; sc1 = bf16(scale + 1). Replaces temporal_pre_norm / channel_pre_norm
 * (tapnext/npu/step8.py:474, :480; numerics tapnext/npu/pack8.py:222-229). */
int mx_rmsnorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* sc1, uint16_t* Y, long ldy, int rows, int D,
               float eps);

/* ============================================================================================ inputs
 * u8 HWC images -> patch rows (c, ky, kx) for the patch-embedding GEMM, zero padded to ldo columns.
 * mode 0: moondream2 normalisation (md2fast.py:148-149); mode 1: TRecViT /127.5 - 1 (tapnext/npu/step8.py:379-383).
 * Replaces the torch permute/div/sub/reshape at md2fast.py:148-149 and the CPU conv input of step8.py:256. */
int mx_patchify_u8(hipStream_t st, const uint8_t* img, uint16_t* out, long ldo, int B, int S, int P, int mode);
/* TRecViT preprocess fused with the patch rows: (B, Hs, Ws, 3) u8 frames -> bilinear resize to S x S
 * (align_corners = False, fp32 pixel values) -> x / 127.5 - 1 -> bf16 rows as mx_patchify_u8 mode 1. Replaces
 * preprocess (F.interpolate + normalisation, tapnext/npu/step8.py:379-383) and the conv input of step8.py:256. */
int mx_resize_patchify_u8(hipStream_t st, const uint8_t* img, int Hs, int Ws, uint16_t* out, long ldo, int B, int S,
                          int P);

/* ============================================================================================ text decoder
 * Partial rotary (dims 0..31) of q and k from fused qkv rows at positions pos0.., q -> q_out [B][H][n][64], rotated k
 * and raw v -> caches [slot][H][ctx][64]; cs = (ctx_table, 16, 2) fp32 (cos, sin). bcast: B = 1 rows to every slot.
 * qkv (ldq % 8 == 0), cs, q_out and the caches 16-byte aligned, else MX_ELAYOUT.
 * Replaces rope_cache / _rope_cache (moondream/gpu/fused.py:5-41; reference rotation fused.py:53-58). */
int mx_rope_kv(hipStream_t st, const uint16_t* qkv, long ldq, const float* cs, uint16_t* q_out, uint16_t* kc,
               uint16_t* vc, int B, int n, int H, int ctx, int pos0, int nslots, int bcast);
/* Batch-1 decode: out1[0:n1] = LN(x)W[0:n1]^T + b; out2 = act2(LN(x)W[n1:N]^T + b) (LN skipped when gamma is null).
 * The M = 1 form of the reference's small-M split-K GEMM (i8gemm_small_launch, i8gemm.hip:555-592) for the fused
 * [qkv | fc1] projection of one token (md2fast.py:173-198). K in {1024, 2048}. */
int mx_ln_gemv2(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta, float eps,
                const uint16_t* W, long ldw, const float* bias, int N, int K, int n1, uint16_t* out1, uint16_t* out2,
                int act2);
/* out = bf16(bf16(W2 g + b2) + bf16(bf16(Wp a + bp) + xres)): the parallel residual of md2fast.py:198
 * (mlp(..., res=lin_res(proj, a, x))) for one token, both GEMVs in one pass. */
int mx_gemv_dual_res(hipStream_t st, const uint16_t* g, const uint16_t* W2, const float* b2, int K2, const uint16_t* a,
                     const uint16_t* Wp, const float* bp, int Kp, const uint16_t* xres, uint16_t* out, int N);
/* W8A8 forms of the two decode GEMVs (the reference's HI8Lin text linears at batch 1, moondream/gpu/hgemm.py:95-137):
 * each workgroup quantises the activation row per token (tgemm.py:81-91), int8 dot products sum exactly in int32,
 * then the fp32 dequant ((acc * s) * sw[n]) + bias[n] and any GELU before one bf16 rounding (i8gemm.hip:181-197).
 * mx_ln_gemv2_i8: LN fused in front (gamma = beta = null: none); Wq int8 (N, ldw bytes, ldw % 16 == 0); K 2048 / 1024.
 * mx_gemv_dual_res_i8: out = bf16(bf16(fc2(g)) + bf16(bf16(proj(a)) + xres)), W2 (N, K2) and Wp (N, Kp) int8
 * contiguous, (K2, Kp) = (8192, 2048) or (4096, 1024). */
int mx_ln_gemv2_i8(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta, float eps,
                   const int8_t* Wq, long ldw, const float* sw, const float* bias, int N, int K, int n1, uint16_t* out1,
                   uint16_t* out2, int act2);
int mx_gemv_dual_res_i8(hipStream_t st, const uint16_t* g, const int8_t* W2, const float* sw2, const float* b2, int K2,
                        const uint16_t* a, const int8_t* Wp, const float* swp, const float* bp, int Kp,
                        const uint16_t* xres, uint16_t* out, int N);
/* LM head: logits = LN(x) W^T + b (bf16; written when logits != null) and one argmax key per workgroup in part
 * (first index wins ties). Replaces the lm_head / lm_small call and the argmax of md2fast.py:212, :281. */
int mx_ln_gemv_argmax(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta, float eps,
                      const uint16_t* W, long ldw, const float* bias, int N, int K, uint16_t* logits,
                      unsigned long long* part, int nparts);
int mx_lm_argmax_nparts(int N);
/* Reduce the argmax keys -> token; tokens[state[0]] = token; state[1] = pos_base + state[0]; state[0]++;
 * x = wte[token]. cap = the steps the caller's buffers hold (tokens[] entries and cache rows past pos_base): at
 * state[0] >= cap nothing is recorded and the state stops advancing, so a step the caller did not stop cannot write
 * past them (the decode attention also clamps its position below ctx). Replaces the host-side argmax + F.embedding
 * of a greedy step (md2fast.py:209). */
int mx_embed_step(hipStream_t st, const unsigned long long* part, int nparts, const uint16_t* wte, int D, int* state,
                  int pos_base, int* tokens, int cap, uint16_t* x);
/* One decode token: rope of q and k at pos = state[1], K/V append at pos, attention over keys 0..pos into out
 * (H * 64): one workgroup per head, 16 waves with a one-pass online softmax each, merged in LDS. S, ws and cnt
 * are unused (ws / cnt may be null; kept for ABI stability). Replaces the SDPA over the KV cache of md2fast.py:185 for one
 * query. */
int mx_decode_attn(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc, int H, int ctx,
                   const int* state, int S, float scale, float* ws, int* cnt, uint16_t* out);
/* The decode step's attention and the parallel residual's fc2 GEMV in one launch (fc2 reads only the fc1 output g),
 * i.e. the attention and parallel residual of md2fast.py:185-198 for one token:
 *  - mx_decode_attn_fc2: the attention of mx_decode_attn on H S workgroups (S splits of each head's keys,
 *    1 <= S <= 8) and y2 = bf16(g W2^T + b2) (W2 (N, K2) contiguous, K2 8192 / 4096) on workgroups of their own.
 *    S = 1 writes attn_out (H 64 bf16); S > 1 writes each split's unnormalised softmax record (M, Lsum, acc[64]) to
 *    part (H S 66 floats) instead.
 *  - mx_gemv_res2: out = bf16(y2 + bf16(bf16(a Wp^T + bp) + xres)) (Wp (N, Kp) contiguous, Kp = 64 H = 2048 / 1024;
 *    out may alias xres), with a = attn_out (S = 1) or merged from part (S > 1).
 * With S = 1 the pair gives mx_decode_attn + mx_gemv_dual_res bit for bit; S > 1 rounds the merged attention output
 * once more in a different order. The _i8 forms take the W8A8 weights and quantise g / a per token inside (the
 * epilogue of mx_gemv_dual_res_i8). */
int mx_decode_attn_fc2(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc, int H, int ctx,
                       const int* state, float scale, int S, float* part, uint16_t* attn_out, const uint16_t* g,
                       const uint16_t* W2, const float* b2, int K2, uint16_t* y2, int N);
int mx_gemv_res2(hipStream_t st, const uint16_t* y2, const uint16_t* a, int S, const float* part, const uint16_t* Wp,
                 const float* bp, int Kp, const uint16_t* xres, uint16_t* out, int N);
int mx_decode_attn_fc2_i8(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc, int H,
                          int ctx, const int* state, float scale, int S, float* part, uint16_t* attn_out,
                          const uint16_t* g, const int8_t* W2, const float* sw2, const float* b2, int K2, uint16_t* y2,
                          int N);
int mx_gemv_res2_i8(hipStream_t st, const uint16_t* y2, const uint16_t* a, int S, const float* part, const int8_t* Wp,
                    const float* swp, const float* bp, int Kp, const uint16_t* xres, uint16_t* out, int N);
/* A whole greedy decode step of the 2048-wide, 32-head (64 dims), 8192-MLP text model in ONE launch: every layer of
 * md2fast.py:173-198 for one token (LN -> [qkv | fc1] + GELU, rope + K/V append at pos = state[1], attention over
 * keys 0..pos, fc2 / proj and the parallel residual), the final LN + LM head + argmax, and mx_embed_step's
 * bookkeeping (tokens[state[0]] = token, state advanced, x = wte[token]; nothing recorded at state[0] >= cap).
 * layers: nl descriptors of mx_decode_mk_layer_bytes() bytes in device memory, each 13 device pointers {ln gamma,
 * ln beta, Wqf = [Wqkv; Wfc1] (14336 x 2048 bf16), bqf (fp32), W2 (2048 x 8192), b2, Wp (2048 x 2048), bp, K cache,
 * V cache (slot 0 of [slot][32][ctx][64]), and three weight-scale pointers used only by mx_decode_step_mk_i8}. logits (V bf16) optional. ll: mx_decode_mk_words() exchange words and
 * ep: 2 words {epoch base, error}, all zeroed once and owned by one decoder; ep[1] != 0 after a step = a wait timed
 * out (the grid exited; zero ll and ep before the next step). The kernel runs mx_decode_mk_grid() workgroups that
 * must all be resident: it refuses (MX_ESHAPE) a device with fewer CUs, and ctx > 1024 or V > 65536.
 * Replaces the per-layer kernel sequence of a greedy step (the reference never decodes, md2fast.py:10-11). */
int mx_decode_step_mk(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g, const uint16_t* lnf_b,
                      const uint16_t* wlm, const float* blm, int V, const uint16_t* wte, const float* cs, float eps,
                      float scale, uint16_t* x, int* state, int pos_base, int* tokens, int cap, uint16_t* logits,
                      uint64_t* ll, uint32_t* ep);
/* The same step with the W8A8 text Linears (the reference's default HI8Lin text path, hgemm.py:95-137): each
 * descriptor's Wqf / W2 / Wp are int8 (the same shapes, one byte per weight, per-row fp32 scales in its last three
 * pointers sqf, sw2, swp, which must not be null); the LN output, g and the attention output are quantised per token
 * (tgemm.py:81-91), the int8 dots summed exactly, and each Linear dequantised as ((acc s_x) s_w) + b with GELU on that
 * fp32 value (i8gemm.hip:181-197); the LM head stays bf16. Replaces the W8A8 per-layer kernel sequence of a step. */
int mx_decode_step_mk_i8(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g,
                         const uint16_t* lnf_b, const uint16_t* wlm, const float* blm, int V, const uint16_t* wte,
                         const float* cs, float eps, float scale, uint16_t* x, int* state, int pos_base, int* tokens,
                         int cap, uint16_t* logits, uint64_t* ll, uint32_t* ep);
int mx_decode_mk_words(void);
int mx_decode_mk_grid(void);
int mx_decode_mk_layer_bytes(void);

/* ============================================================================================ TRecViT recurrence
 * One streamed frame of conv_1d + block-diagonal gates + RG-LRU + y-gate (numerics of tapnext/npu/pack8.py:253-279
 * ssm_ref and tapnext/npu/r9/cpuemu.py:33-47 RGLRU.forward): taps x0 (current) .. x3 (t-3), h fp32 updated in place,
 * z = bf16(bf16(h) * yg). frame: device int, 0 = first frame of the video. Replaces the NPU EW core's ew_ssm
 * (tapnext/npu/ew8.cc:1351, :1556-1578) and the torch recurrent_block of model.step. */
int mx_ssm_step(hipStream_t st, const uint16_t* x0, const uint16_t* x1, const uint16_t* x2, const uint16_t* x3,
                long ld_x, const uint16_t* yg, long ld_y, const uint16_t* conv_w, const uint16_t* conv_b,
                const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT, const uint16_t* ba, const uint16_t* sp,
                const int* frame, float* h, uint16_t* z, long ld_z, int T, int C);
/* The same step for a moving crop of patch tokens with the state indexed by absolute patch (the shifted crop of
 * tapnext/crop-study/crop_study.py:147-185, CropTracker(shift=True)): x0 / yg / z hold the launch's T tokens; h, the
 * history taps x1..x3 (stride ld_x) and xsave (this frame's history slot, stride ld_save, receives x0) are addressed
 * at state row rows[t] (distinct rows < srows). stamps [2][srows] {frame entered, last frame present} (set to
 * {-8, -8} at a video start) replace the reference's zero-then-write of the state buffers: a row absent on the
 * previous frame starts from zero state, history tap k is used only if the row was present since frame t - k. */
int mx_ssm_step_rows(hipStream_t st, const uint16_t* x0, const uint16_t* x1, const uint16_t* x2, const uint16_t* x3,
                     long ld_x, const uint16_t* yg, long ld_y, const uint16_t* conv_w, const uint16_t* conv_b,
                     const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT, const uint16_t* ba,
                     const uint16_t* sp, const int* frame, float* h, uint16_t* z, long ld_z, int T, int C,
                     const int* rows, int* stamps, int srows, uint16_t* xsave, long ld_save);
/* The RG-LRU layer alone: TAPNext's RGLRU.forward(x, h0) -> (y, h) (tapnext/npu/r9/cpuemu.py:33-47, the layer the
 * reference swaps at :110-116; the Python binding is refbind.rglru_forward / trecvit.RGLRU). x [T][ld_x] bf16 is
 * the layer's input (the temporal conv's output), h0 [T][C] fp32 the state or NULL on the first frame (then
 * h = bf(x * bf(sigmoid(gx)))); h [T][C] fp32 receives the new state (h == h0 updates in place) and y [T][ld_y]
 * bf16 = bf(h). Gates as in mx_ssm_step (wxT / waT [H][64 out][64 in], bx / ba [C], sp = bf16(softplus(a_param))).
 * x and the gate weights 16-byte aligned, ld_x % 8 == 0, C % 64 == 0. */
int mx_rglru_step(hipStream_t st, const uint16_t* x, long ld_x, const float* h0, const uint16_t* wxT,
                  const uint16_t* bx, const uint16_t* waT, const uint16_t* ba, const uint16_t* sp, float* h,
                  uint16_t* y, long ld_y, int T, int C);
/* Clip form of the same recurrence: per-frame affine maps h -> A h + B for F frames (x_stack = 3 history frames then
 * the F frames, frame stride fs_x), then the time scan. No reference counterpart (the reference only streams):
 * a frame-parallel restatement of the same recurrence. */
int mx_ssm_prep(hipStream_t st, const uint16_t* x_stack, long ld_x, long fs_x, const uint16_t* conv_w,
                const uint16_t* conv_b, const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT, const uint16_t* ba,
                const uint16_t* sp, const int* frame, float* A, float* B, int F, int T, int C);
int mx_rglru_scan(hipStream_t st, const float* A, const float* B, float* h, int F, int T, int C, const uint16_t* yg,
                  long ld_y, long fs_y, uint16_t* z, long ld_z, long fs_z);

/* ============================================================================================ TAPNext heads
 * model.heads (tapnext/npu/step8.py:327-362, heads_np; the torch module it restates at step8.py:364-376): per query
 * row, the coordinate head and the visibility head, each Linear(D,H) -> LayerNorm -> GELU erf -> Linear(H,H) ->
 * LayerNorm -> GELU erf -> Linear(H,NO) in fp32, and the coordinate head's two n-bin halves read out as
 * E[i] under softmax(0.5 logits) masked to |argmax - i| <= radius, renormalised, + 0.5.
 * Weight blob per head (fp32): W0^T [D][H] | b0 | g0 | beta0 | W1^T [H][H] | b1 | g1 | beta1 | W2^T [H][NO] | b2.
 * x: bf16 rows (stride ldx); outputs fp32 tracks (Q, 2), logits (Q, NOC) stride ldl, vis (Q). D and H multiples
 * of 32, H <= 256, NOC even and <= 512. */
long mx_track_head_blob_elems(int D, int H, int NO);
int mx_track_heads(hipStream_t st, const uint16_t* x, long ldx, int Q, int D, int H, const float* cblob, int NOC,
                   float ce0, float ce1, const float* vblob, float ve0, float ve1, int radius, float* tracks,
                   float* logits, long ldl, float* vis);

/* ============================================================================================ misc
 * p[0] += v on the stream: the frame counter a captured frame graph advances (no counterpart in the reference,
 * whose frame index lives on the host: tapnext/npu/step8.py:232-249 set_first / reset). */
int mx_counter_add(hipStream_t st, int* p, int v);

#ifdef __cplusplus
}
#endif
#endif /* SHMAXX_H */
