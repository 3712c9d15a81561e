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

}  // namespace

extern "C" int mx_patchify_u8(hipStream_t st, const uint8_t* img, uint16_t* out, long ldo, int B, int S, int P,
                              int mode) {
  if (!img || !out) return MX_ENULL;
  if (B < 1 || P < 1 || S % P || ldo < 3L * P * P || mode < 0 || mode > 1) return MX_ESHAPE;
  const long total = (long)B * (S / P) * (S / P) * ldo;
  const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  hipLaunchKernelGGL(patchify_kernel, dim3(blocks), dim3(256), 0, st, img, out, ldo, B, S, P, mode);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
