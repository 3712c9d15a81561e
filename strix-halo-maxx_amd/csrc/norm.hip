// Row normalisations (one 64-wide wave per row, 16-byte vector loads, fp32 statistics).
//  * LayerNorm  y = bf16((x - mean) * rsqrt(var + eps) * gamma + beta)   (torch F.layer_norm on bf16: fp32 inside,
//    one rounding at the end; biased variance)
//  * RMSNorm in the TRecViT form with torch's bf16 op-by-op rounding:
//      s = sum_fp32 bf16(x^2); ms = bf16(s / D); rstd = bf16(1 / sqrt(bf16(ms + eps))); y = bf16(bf16(x * rstd) * sc1)
//    where sc1 = bf16(scale + 1) is supplied by the caller.
#include "common.h"

namespace {

// Both kernels issue every load of the row (and gamma / beta / sc1) in one straight run before any arithmetic, and
// run the arithmetic on every chunk: a row is latency-bound, and conditional loads or loads after the statistics
// would cost further memory round trips. Chunks past the row's end reload its last chunk, add zeros to the sums and
// store nothing.
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
  u32x4 q[MAXC], gv[MAXC], ev[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = min(lane + 64 * i, nch - 1);
    q[i] = *reinterpret_cast<const u32x4*>(x + c * 8);
    gv[i] = *reinterpret_cast<const u32x4*>(gamma + c * 8);
    ev[i] = *reinterpret_cast<const u32x4*>(beta + c * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  float v[MAXC][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int e = 0; e < 4; e++) { v[i][2 * e] = lo_bf(q[i][e]); v[i][2 * e + 1] = hi_bf(q[i][e]); }
#pragma unroll
    for (int e = 0; e < 8; e++) s += ok ? v[i][e] : 0.f;
  }
  const float mean = wave_sum(s) / (float)D;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float d = v[i][e] - mean;
      ss += ok ? d * d : 0.f;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
  uint16_t* y = Y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float y0 = (v[i][2 * e] - mean) * rstd * lo_bf(gv[i][e]) + lo_bf(ev[i][e]);
      const float y1 = (v[i][2 * e + 1] - mean) * rstd * hi_bf(gv[i][e]) + hi_bf(ev[i][e]);
      o[e] = pack2(y0, y1);
    }
    if (c < nch) *reinterpret_cast<u32x4*>(y + c * 8) = o;
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
  u32x4 q[MAXC], gv[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = min(lane + 64 * i, nch - 1);
    q[i] = *reinterpret_cast<const u32x4*>(x + c * 8);
    gv[i] = *reinterpret_cast<const u32x4*>(sc1 + c * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  float v[MAXC][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int e = 0; e < 4; e++) { v[i][2 * e] = lo_bf(q[i][e]); v[i][2 * e + 1] = hi_bf(q[i][e]); }
#pragma unroll
    for (int e = 0; e < 8; e++) s += ok ? rbf(v[i][e] * v[i][e]) : 0.f;
  }
  const float ms = rbf(wave_sum(s) / (float)D);
  const float rstd = rbf(1.0f / sqrtf(rbf(ms + eps)));
  uint16_t* y = Y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float y0 = rbf(v[i][2 * e] * rstd) * lo_bf(gv[i][e]);
      const float y1 = rbf(v[i][2 * e + 1] * rstd) * hi_bf(gv[i][e]);
      o[e] = pack2(y0, y1);
    }
    if (c < nch) *reinterpret_cast<u32x4*>(y + c * 8) = o;
  }
}

// Split-K reduction + bias + residual, then LayerNorm, one wave per row:
//   x = bf16(bf16(sum_s P[s] + bias) + R)      (the Linear output rounded to bf16, then the fp32 residual add,
//                                               rounded once more: torch's order for `linear(...) + res` in bf16)
//   y = LayerNorm(x) as in layernorm_kernel (skipped when gamma is null), or with RMS the TRecViT RMSNorm of
//   rmsnorm_kernel (gamma = sc1 = bf16(scale + 1), beta unused)
// The partials are added in split order, so the result does not depend on scheduling.
template <int MAXC, int NS, bool RMS = false>
__global__ __launch_bounds__(256) void residual_layernorm_kernel(
    const float* __restrict__ P, long p_split, long ldp, const float* __restrict__ bias,
    const uint16_t* __restrict__ R, long ldr, uint16_t* __restrict__ Xo, long ldxo, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ Y, long ldy, int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = D >> 3;
  // Every load of the row, gamma and beta included, is issued before any arithmetic, in one straight run: the row is
  // latency-bound, not bandwidth-bound, and conditional loads would let the compiler wait for some of them before
  // issuing the rest. Chunks past the row's end load its last chunk and a missing bias / gamma / beta loads from
  // another valid row; neither is used.
  f32x4 pv[MAXC][NS][2];
  u32x4 rv[MAXC], gv[MAXC], ev[MAXC];
  f32x4 bv[MAXC][2];
  const float* bsrc = bias ? bias : P;
  const uint16_t* gsrc = gamma ? gamma : R;
  const uint16_t* esrc = beta ? beta : R;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = min(lane + 64 * i, nch - 1);
    const float* p = P + (long)row * ldp + c * 8;
#pragma unroll
    for (int sp = 0; sp < NS; sp++) {
      pv[i][sp][0] = *reinterpret_cast<const f32x4*>(p + sp * p_split);
      pv[i][sp][1] = *reinterpret_cast<const f32x4*>(p + sp * p_split + 4);
    }
    rv[i] = *reinterpret_cast<const u32x4*>(R + (long)row * ldr + c * 8);
    bv[i][0] = *reinterpret_cast<const f32x4*>(bsrc + c * 8);
    bv[i][1] = *reinterpret_cast<const f32x4*>(bsrc + c * 8 + 4);
    gv[i] = *reinterpret_cast<const u32x4*>(gsrc + c * 8);
    ev[i] = *reinterpret_cast<const u32x4*>(esrc + c * 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // all of them before the first use
  // The arithmetic runs on every chunk (a branch around it would let the loads sink into it); chunks past the row's
  // end add zeros to the row sums and store nothing.
  float v[MAXC][8];
  float s = 0.f;
  const bool hb = bias != nullptr;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    const bool ok = c < nch;
    float a[8];
#pragma unroll
    for (int e = 0; e < 4; e++) { a[e] = pv[i][0][0][e]; a[4 + e] = pv[i][0][1][e]; }
#pragma unroll
    for (int sp = 1; sp < NS; sp++)
#pragma unroll
      for (int e = 0; e < 4; e++) { a[e] += pv[i][sp][0][e]; a[4 + e] += pv[i][sp][1][e]; }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      a[e] = hb ? a[e] + bv[i][0][e] : a[e];
      a[4 + e] = hb ? a[4 + e] + bv[i][1][e] : a[4 + e];
    }
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[i][2 * e] = rbf(rbf(a[2 * e]) + lo_bf(rv[i][e]));
      v[i][2 * e + 1] = rbf(rbf(a[2 * e + 1]) + hi_bf(rv[i][e]));
      o[e] = pack2(v[i][2 * e], v[i][2 * e + 1]);
    }
    if (ok) *reinterpret_cast<u32x4*>(Xo + (long)row * ldxo + c * 8) = o;
#pragma unroll
    for (int e = 0; e < 8; e++) s += ok ? (RMS ? rbf(v[i][e] * v[i][e]) : v[i][e]) : 0.f;
  }
  if (!gamma) return;
  if constexpr (RMS) {  // s = sum_fp32 bf16(x^2); rstd = bf16(1 / sqrt(bf16(bf16(s / D) + eps))); y = bf16(bf16(x rstd) sc1)
    const float ms = rbf(wave_sum(s) / (float)D);
    const float rstd = rbf(1.0f / sqrtf(rbf(ms + eps)));
    uint16_t* y = Y + (long)row * ldy;
#pragma unroll
    for (int i = 0; i < MAXC; i++) {
      const int c = lane + 64 * i;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++)
        o[e] = pack2(rbf(v[i][2 * e] * rstd) * lo_bf(gv[i][e]), rbf(v[i][2 * e + 1] * rstd) * hi_bf(gv[i][e]));
      if (c < nch) *reinterpret_cast<u32x4*>(y + c * 8) = o;
    }
    return;
  }
  const float mean = wave_sum(s) / (float)D;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float d = v[i][e] - mean;
      ss += ok ? d * d : 0.f;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
  uint16_t* y = Y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int c = lane + 64 * i;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float y0 = (v[i][2 * e] - mean) * rstd * lo_bf(gv[i][e]) + lo_bf(ev[i][e]);
      const float y1 = (v[i][2 * e + 1] - mean) * rstd * hi_bf(gv[i][e]) + hi_bf(ev[i][e]);
      o[e] = pack2(y0, y1);
    }
    if (c < nch) *reinterpret_cast<u32x4*>(y + c * 8) = o;
  }
}

int check(const void* X, long ldx, const void* Y, long ldy, int rows, int D) {
  if (!X || !Y) return MX_ENULL;
  if (rows < 1 || D < 8 || D % 8 || D > 8192 || ldx % 8 || ldy % 8 || ldx < D || ldy < D) return MX_ESHAPE;
  if (((uintptr_t)X | (uintptr_t)Y) & 15) return MX_ELAYOUT;
  return MX_OK;
}

// residual_layernorm_kernel for a validated call: chunks per lane from D (<= 2048), splits 1..4.
template <bool RMS>
int launch_residual_norm(hipStream_t st, const float* P, int nsplit, long p_split, long ldp, const float* bias,
                         const uint16_t* R, long ldr, uint16_t* Xo, long ldxo, const uint16_t* gamma,
                         const uint16_t* beta, uint16_t* Y, long ldy, int rows, int D, float eps) {
  dim3 g((rows + 3) / 4);
  const int nch = D / 8;
#define L2_(C, NS) hipLaunchKernelGGL((residual_layernorm_kernel<C, NS, RMS>), g, dim3(256), 0, st, P, p_split, ldp, bias, R, ldr, Xo, ldxo, gamma, beta, Y, ldy, rows, D, eps)
#define L_(C) switch (nsplit) { case 1: L2_(C, 1); break; case 2: L2_(C, 2); break; case 3: L2_(C, 3); break; default: L2_(C, 4); }
  if (nch <= 128) { L_(2); }
  else if (nch <= 192) { L_(3); }
  else if (nch <= 256) { L_(4); }
  else return MX_ESHAPE;
#undef L2_
#undef L_
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
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

// x = bf16(bf16(sum_s P[s] + bias) + R) -> Xo; y = LayerNorm(x; gamma, beta, eps) -> Y (skipped if gamma is null).
// P: nsplit fp32 partial sums (split stride p_split, row stride ldp), e.g. from mx_gemm_bf16_partial. bias: fp32 or
// null. Fuses the epilogue of a residual Linear with the LayerNorm that consumes its output (the reference runs them
// as `x = x + proj(a)` then `ln2(x)`, moondream/gpu/md2fast.py:152-157).
extern "C" int mx_residual_layernorm(hipStream_t st, const float* P, int nsplit, long p_split, long ldp,
                                     const float* bias, const uint16_t* R, long ldr, uint16_t* Xo, long ldxo,
                                     const uint16_t* gamma, const uint16_t* beta, uint16_t* Y, long ldy, int rows,
                                     int D, float eps) {
  if (!P || !R || !Xo) return MX_ENULL;
  if (nsplit < 1 || rows < 1 || D < 8 || D % 8 || D > 2048) return MX_ESHAPE;
  if (ldp % 4 || ldp < D || ldr % 8 || ldr < D || ldxo % 8 || ldxo < D || (nsplit > 1 && (p_split % 4 || p_split < (long)rows * ldp)))
    return MX_ESHAPE;
  if ((((uintptr_t)P | (uintptr_t)R | (uintptr_t)Xo) & 15) || (bias && ((uintptr_t)bias & 15))) return MX_ELAYOUT;
  if (gamma) {
    if (!beta || !Y) return MX_ENULL;
    if (ldy % 8 || ldy < D) return MX_ESHAPE;
    if (((uintptr_t)gamma | (uintptr_t)beta | (uintptr_t)Y) & 15) return MX_ELAYOUT;
  }
  if (nsplit > 4) return MX_ESHAPE;
  return launch_residual_norm<false>(st, P, nsplit, p_split, ldp, bias, R, ldr, Xo, ldxo, gamma, beta, Y, ldy, rows,
                                     D, eps);
}

// x = bf16(bf16(sum_s P[s] + bias) + R) -> Xo; y = the TRecViT RMSNorm of x (sc1 = bf16(scale + 1)) -> Y. The
// epilogue of a residual Linear fused with the RMSNorm that reads its output (tapnext/npu/step8.py:470-488: the
// ssm block's linear_out + x, then the channel pre-norm; the ViT block's mlp3 + x2, then the next block's temporal
// pre-norm). Same operands and rules as mx_residual_layernorm, sc1 in place of gamma / beta (required).
extern "C" int mx_residual_rmsnorm(hipStream_t st, const float* P, int nsplit, long p_split, long ldp,
                                   const float* bias, const uint16_t* R, long ldr, uint16_t* Xo, long ldxo,
                                   const uint16_t* sc1, uint16_t* Y, long ldy, int rows, int D, float eps) {
  if (!P || !R || !Xo || !sc1 || !Y) return MX_ENULL;
  if (nsplit < 1 || nsplit > 4 || rows < 1 || D < 8 || D % 8 || D > 2048) return MX_ESHAPE;
  if (ldp % 4 || ldp < D || ldr % 8 || ldr < D || ldxo % 8 || ldxo < D || ldy % 8 || ldy < D ||
      (nsplit > 1 && (p_split % 4 || p_split < (long)rows * ldp)))
    return MX_ESHAPE;
  if ((((uintptr_t)P | (uintptr_t)R | (uintptr_t)Xo | (uintptr_t)sc1 | (uintptr_t)Y) & 15) ||
      (bias && ((uintptr_t)bias & 15)))
    return MX_ELAYOUT;
  return launch_residual_norm<true>(st, P, nsplit, p_split, ldp, bias, R, ldr, Xo, ldxo, sc1, nullptr, Y, ldy, rows,
                                    D, eps);
}
