/* C ABI of libshmaxx.so: the MI355X (gfx950) kernels of the strix-halo-maxx hot path.
 *
 * Conventions (same style as the reference's launchers, moondream/gpu/hip/i8gemm.hip:478-595, attn.hip:433-462):
 *  - plain C types only: hipStream_t, raw device pointers, element counts/strides (in elements, not bytes);
 *  - bf16 tensors are passed as uint16_t* bit patterns, fp32 as float*;
 *  - every entry point launches asynchronously on the given stream, never allocates, frees or synchronises, and
 *    returns 0 or a negative status:
 *      -1 unknown config / head dim / mode   -2 unsupported shape or stride   -3 workspace too small
 *      -4 pointer alignment / layout         -5 HIP launch failed             -6 required pointer is null
 *  - shapes are validated on the host before any launch (the *_check functions run that validation alone).
 */
#ifndef SHMAXX_H
#define SHMAXX_H
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------- GEMM (MFMA)
 * C[M,N] = epi(A[M,K] . W[N,K]^T + bias[N]); epi: act (0 none, 1 GELU-tanh, 2 GELU-erf) applied to the bf16-rounded
 * linear output, then "+ R" (R row = m % r_rows when r_rows > 0, else m), each step rounded to bf16.
 * Requirements: K % 8 == 0, lda/ldw % 8 == 0, A/W 16-byte aligned, N % 4 == 0, ldc/ldr % 4 == 0, bias 16-byte aligned.
 * cfg < 0 lets the library pick the tile; 0..mx_gemm_ncfg()-1 forces one.
 * Replaces: bf16gemm_launch (moondream/gpu/hip/i8gemm.hip:534-552, bound in hgemm.py:28), whose act flag is the
 * `gelu` argument and whose residual the reference adds outside (md2fast.py:64-67). */
int mx_gemm_bf16(hipStream_t st, int cfg, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
                 const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int K, int act);
/* Host-only validation of an mx_gemm_bf16 call. Replaces the shape checks at i8gemm.hip:535. */
int mx_gemm_check(int cfg, const void* A, long lda, const void* W, long ldw, const void* bias, const void* R, long ldr,
                  const void* C, long ldc, int M, int N, int K, int act);
/* Tile config the library would pick for (M, N, K). Replaces pick_cfg's FIXED table (hgemm.py:47-51). */
int mx_gemm_pick(int M, int N, int K);
/* Number of tile configs / the (BM, BN) tile of one. Replaces bf16gemm_ncfg (i8gemm.hip:553). */
int mx_gemm_ncfg(void);
int mx_gemm_cfg_tile(int cfg, int* bm, int* bn);

/* ---------------------------------------------------------------------------------------------- attention
 * O[b, i, h*D + d] = softmax(scale * Q K^T) V over visible keys; key j visible to query i iff j < Tk and
 * (j < causal_from || j <= qpos0 + i). D in {64, 72}. Q/K/V/O addressed as base + b*s_b + h*s_h + t*s_t + d.
 * Replaces: attn_fwd2 + vtranspose (moondream/gpu/hip/attn.hip:442-451, :275-288; bound in hattn.py:11-14), which
 * are mask-free and batch 1; the masked prompt prefill (md2fast.py:132-136, :185) used torch SDPA there. */
int mx_sdpa(hipStream_t st, const uint16_t* Q, long sq_b, long sq_h, long sq_t, const uint16_t* K, long sk_b,
            long sk_h, long sk_t, const uint16_t* V, long sv_b, long sv_h, long sv_t, uint16_t* O, long so_b, long so_h,
            long so_t, int B, int H, int Tq, int Tk, int D, float scale, int qpos0, int causal_from);
int mx_sdpa_check(const void* Q, long sq_t, const void* K, long sk_t, const void* V, long sv_t, const void* O,
                  long so_t, int B, int H, int Tq, int Tk, int D);

/* ---------------------------------------------------------------------------------------------- norms
 * LayerNorm over rows of D (fp32 statistics, one rounding). Replaces F.layer_norm in _ln (md2fast.py:43-44) and the
 * TRecViT ln_1 / ln_2 / encoder_norm (tapnext/npu/pack8.py:232-238 restates its numerics). */
int mx_layernorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* gamma, const uint16_t* beta, uint16_t* Y,
                 long ldy, int rows, int D, float eps);
/* TRecViT RMSNorm with torch's bf16 rounding; sc1 = bf16(scale + 1). Replaces temporal_pre_norm / channel_pre_norm
 * (tapnext/npu/step8.py:474, :480; numerics pack8.py:222-229). */
int mx_rmsnorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* sc1, uint16_t* Y, long ldy, int rows, int D,
               float eps);

/* ---------------------------------------------------------------------------------------------- input
 * u8 HWC images -> patch rows (c, ky, kx) for the patch-embedding GEMM, zero padded to ldo columns.
 * mode 0: moondream2 normalisation (md2fast.py:148-149); mode 1: TRecViT /127.5 - 1 (step8.py:379-383).
 * Replaces the torch permute/div/sub/reshape sequence at md2fast.py:148-149 and the CPU conv input of step8.py:256. */
int mx_patchify_u8(hipStream_t st, const uint8_t* img, uint16_t* out, long ldo, int B, int S, int P, int mode);

#ifdef __cplusplus
}
#endif
#endif /* SHMAXX_H */
