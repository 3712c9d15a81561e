// Image -> patch-row matrix for the patch-embedding GEMM (a stride = kernel conv is a GEMM over patches).
//   img u8 [B][S][S][3] (HWC)  ->  out bf16 [B * G * G][ldo], G = S / P, column k = c * P * P + ky * P + kx
//   (the (c, ky, kx) order of a Conv2d weight reshaped to [out, 3 * P * P]); columns K .. ldo-1 are written as 0 so
//   the GEMM can use a K padded to a multiple of 8.
// Normalisation modes:
//   0  moondream2:  bf16 ops in sequence  x = bf16(u8) / 255 -> bf16 ; - 0.5 -> bf16 ; / 0.5 (exact)
//   1  TRecViT:     fp32  x = u8 / 127.5 - 1, then one rounding to bf16
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void patchify_kernel(const uint8_t* __restrict__ img, uint16_t* __restrict__ out,
                                                       long ldo, int B, int S, int P, int mode) {
  const int G = S / P, K = 3 * P * P;
  const long total = (long)B * G * G * ldo;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    const long row = i / ldo;
    const int k = (int)(i % ldo);
    uint16_t v = 0;
    if (k < K) {
      const int b = (int)(row / (G * G)), p = (int)(row % (G * G));
      const int gy = p / G, gx = p % G;
      const int c = k / (P * P), r = k % (P * P), ky = r / P, kx = r % P;
      const float u = (float)img[(((long)b * S + gy * P + ky) * S + gx * P + kx) * 3 + c];
      if (mode == 0) {
        const float a = rbf(u / 255.0f);
        v = f2bf(rbf(a - 0.5f) * 2.0f);
      } else {
        v = f2bf(__fsub_rn(__fdiv_rn(u, 127.5f), 1.0f));
      }
    }
    out[i] = v;
  }
}

// Source coordinate of output index d for a bilinear resize, align_corners = False: s = scale (d + 0.5) - 0.5
// clamped at 0; i0 = min(floor(s), n - 1), i1 = i0 + 1 unless i0 is the last index; l1 = clamp(s - i0, 0, 1),
// l0 = 1 - l1 (fp32 throughout, the arithmetic of torch's CPU upsample_bilinear2d).
__device__ __forceinline__ void src_index(float scale, int d, int n, int& i0, int& i1, float& l0, float& l1) {
  float s = __fsub_rn(__fmul_rn(scale, __fadd_rn((float)d, 0.5f)), 0.5f);
  s = s < 0.f ? 0.f : s;
  i0 = min((int)floorf(s), n - 1);
  i1 = i0 + (i0 < n - 1 ? 1 : 0);
  l1 = fminf(fmaxf(__fsub_rn(s, (float)i0), 0.f), 1.f);
  l0 = __fsub_rn(1.f, l1);
}

// TRecViT preprocess + patchify in one pass: img u8 [B][Hs][Ws][3] -> bilinear resize to S x S on the fp32 pixel
// values -> x / 127.5 - 1 -> bf16 patch rows (same output layout as patchify_kernel). The four taps are weighted by
// the products of the row and column weights and summed in the order (0,0), (0,1), (1,0), (1,1).
__global__ __launch_bounds__(256) void resize_patchify_kernel(const uint8_t* __restrict__ img, int Hs, int Ws,
                                                              uint16_t* __restrict__ out, long ldo, int B, int S,
                                                              int P) {
  const int G = S / P, K = 3 * P * P;
  const float sy = __fdiv_rn((float)Hs, (float)S), sx = __fdiv_rn((float)Ws, (float)S);
  const long total = (long)B * G * G * ldo;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    const long row = i / ldo;
    const int k = (int)(i % ldo);
    uint16_t v = 0;
    if (k < K) {
      const int b = (int)(row / (G * G)), p = (int)(row % (G * G));
      const int gy = p / G, gx = p % G;
      const int c = k / (P * P), r = k % (P * P), ky = r / P, kx = r % P;
      int y0, y1, x0, x1;
      float hy0, hy1, wx0, wx1;
      src_index(sy, gy * P + ky, Hs, y0, y1, hy0, hy1);
      src_index(sx, gx * P + kx, Ws, x0, x1, wx0, wx1);
      const uint8_t* base = img + (long)b * Hs * Ws * 3 + c;
      const float p00 = base[((long)y0 * Ws + x0) * 3], p01 = base[((long)y0 * Ws + x1) * 3];
      const float p10 = base[((long)y1 * Ws + x0) * 3], p11 = base[((long)y1 * Ws + x1) * 3];
      const float w00 = __fmul_rn(hy0, wx0), w01 = __fmul_rn(hy0, wx1);
      const float w10 = __fmul_rn(hy1, wx0), w11 = __fmul_rn(hy1, wx1);
      const float val = __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(p00, w00), __fmul_rn(p01, w01)), __fmul_rn(p10, w10)),
                                  __fmul_rn(p11, w11));
      v = f2bf(__fsub_rn(__fdiv_rn(val, 127.5f), 1.0f));
    }
    out[i] = v;
  }
}

}  // namespace

// (B, Hs, Ws, 3) u8 frames -> bilinear resize to S x S (align_corners = False) -> / 127.5 - 1 -> bf16 patch rows
// [B * (S/P)^2][ldo], (c, ky, kx) column order, columns 3 P^2 .. ldo - 1 zero. The TRecViT preprocess
// (tapnext/npu/step8.py:379-383) fused with the patch-conv input (step8.py:256).
extern "C" int mx_resize_patchify_u8(hipStream_t st, const uint8_t* img, int Hs, int Ws, uint16_t* out, long ldo,
                                     int B, int S, int P) {
  if (!img || !out) return MX_ENULL;
  if (B < 1 || P < 1 || S < P || S % P || Hs < 1 || Ws < 1 || Hs > 16384 || Ws > 16384 || ldo < 3L * P * P)
    return MX_ESHAPE;
  const long total = (long)B * (S / P) * (S / P) * ldo;
  const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  hipLaunchKernelGGL(resize_patchify_kernel, dim3(blocks), dim3(256), 0, st, img, Hs, Ws, out, ldo, B, S, P);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_patchify_u8(hipStream_t st, const uint8_t* img, uint16_t* out, long ldo, int B, int S, int P,
                              int mode) {
  if (!img || !out) return MX_ENULL;
  if (B < 1 || P < 1 || S % P || ldo < 3L * P * P || mode < 0 || mode > 1) return MX_ESHAPE;
  const long total = (long)B * (S / P) * (S / P) * ldo;
  const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  hipLaunchKernelGGL(patchify_kernel, dim3(blocks), dim3(256), 0, st, img, out, ldo, B, S, P, mode);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
