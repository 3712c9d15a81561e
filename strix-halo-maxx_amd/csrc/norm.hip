// Row normalisations (one 64-wide wave per row, 16-byte vector loads, fp32 statistics).
//  * LayerNorm  y = bf16((x - mean) * rsqrt(var + eps) * gamma + beta)   (torch F.layer_norm on bf16: fp32 inside,
//    one rounding at the end; biased variance)
//  * RMSNorm in the TRecViT form with torch's bf16 op-by-op rounding:
//      s = sum_fp32 bf16(x^2); ms = bf16(s / D); rstd = bf16(1 / sqrt(bf16(ms + eps))); y = bf16(bf16(x * rstd) * sc1)
//    where sc1 = bf16(scale + 1) is supplied by the caller.
#include "common.h"

namespace {

template <int MAXC>
__global__ __launch_bounds__(256) void layernorm_kernel(const uint16_t* __restrict__ X, long ldx,
                                                        const uint16_t* __restrict__ gamma,
                                                        const uint16_t* __restrict__ beta, uint16_t* __restrict__ Y,
                                                        long ldy, int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = D >> 3;
  const uint16_t* x = X + (long)row * ldx;
  float v[MAXC][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(x + c * 8);
#pragma unroll
      for (int e = 0; e < 4; e++) { v[i][2 * e] = lo_bf(q[e]); v[i][2 * e + 1] = hi_bf(q[e]); }
#pragma unroll
      for (int e = 0; e < 8; e++) s += v[i][e];
    }
  }
  const float mean = wave_sum(s) / (float)D;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; e++) { const float d = v[i][e] - mean; ss += d * d; }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
  uint16_t* y = Y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const u32x4 g = *reinterpret_cast<const u32x4*>(gamma + c * 8);
      const u32x4 bb = *reinterpret_cast<const u32x4*>(beta + c * 8);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float y0 = (v[i][2 * e] - mean) * rstd * lo_bf(g[e]) + lo_bf(bb[e]);
        const float y1 = (v[i][2 * e + 1] - mean) * rstd * hi_bf(g[e]) + hi_bf(bb[e]);
        o[e] = pack2(y0, y1);
      }
      *reinterpret_cast<u32x4*>(y + c * 8) = o;
    }
  }
}

template <int MAXC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ X, long ldx,
                                                      const uint16_t* __restrict__ sc1, uint16_t* __restrict__ Y,
                                                      long ldy, int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = D >> 3;
  const uint16_t* x = X + (long)row * ldx;
  float v[MAXC][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(x + c * 8);
#pragma unroll
      for (int e = 0; e < 4; e++) { v[i][2 * e] = lo_bf(q[e]); v[i][2 * e + 1] = hi_bf(q[e]); }
#pragma unroll
      for (int e = 0; e < 8; e++) s += rbf(v[i][e] * v[i][e]);
    }
  }
  const float ms = rbf(wave_sum(s) / (float)D);
  const float rstd = rbf(1.0f / sqrtf(rbf(ms + eps)));
  uint16_t* y = Y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const u32x4 g = *reinterpret_cast<const u32x4*>(sc1 + c * 8);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float y0 = rbf(v[i][2 * e] * rstd) * lo_bf(g[e]);
        const float y1 = rbf(v[i][2 * e + 1] * rstd) * hi_bf(g[e]);
        o[e] = pack2(y0, y1);
      }
      *reinterpret_cast<u32x4*>(y + c * 8) = o;
    }
  }
}

int check(const void* X, long ldx, const void* Y, long ldy, int rows, int D) {
  if (!X || !Y) return MX_ENULL;
  if (rows < 1 || D < 8 || D % 8 || D > 8192 || ldx % 8 || ldy % 8 || ldx < D || ldy < D) return MX_ESHAPE;
  if (((uintptr_t)X | (uintptr_t)Y) & 15) return MX_ELAYOUT;
  return MX_OK;
}

}  // namespace

extern "C" int mx_layernorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* gamma, const uint16_t* beta,
                            uint16_t* Y, long ldy, int rows, int D, float eps) {
  int rc = check(X, ldx, Y, ldy, rows, D);
  if (rc) return rc;
  if (!gamma || !beta) return MX_ENULL;
  if (((uintptr_t)gamma | (uintptr_t)beta) & 15) return MX_ELAYOUT;
  dim3 g((rows + 3) / 4);
  const int nch = D / 8;
  if (nch <= 128) hipLaunchKernelGGL(layernorm_kernel<2>, g, dim3(256), 0, st, X, ldx, gamma, beta, Y, ldy, rows, D, eps);
  else if (nch <= 256) hipLaunchKernelGGL(layernorm_kernel<4>, g, dim3(256), 0, st, X, ldx, gamma, beta, Y, ldy, rows, D, eps);
  else hipLaunchKernelGGL(layernorm_kernel<16>, g, dim3(256), 0, st, X, ldx, gamma, beta, Y, ldy, rows, D, eps);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_rmsnorm(hipStream_t st, const uint16_t* X, long ldx, const uint16_t* sc1, uint16_t* Y, long ldy,
                          int rows, int D, float eps) {
  int rc = check(X, ldx, Y, ldy, rows, D);
  if (rc) return rc;
  if (!sc1) return MX_ENULL;
  if ((uintptr_t)sc1 & 15) return MX_ELAYOUT;
  dim3 g((rows + 3) / 4);
  const int nch = D / 8;
  if (nch <= 128) hipLaunchKernelGGL(rmsnorm_kernel<2>, g, dim3(256), 0, st, X, ldx, sc1, Y, ldy, rows, D, eps);
  else if (nch <= 256) hipLaunchKernelGGL(rmsnorm_kernel<4>, g, dim3(256), 0, st, X, ldx, sc1, Y, ldy, rows, D, eps);
  else hipLaunchKernelGGL(rmsnorm_kernel<16>, g, dim3(256), 0, st, X, ldx, sc1, Y, ldy, rows, D, eps);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
