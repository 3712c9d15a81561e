// Row-wise int8 quantisation for the W8A8 text linears, one 256-thread workgroup per row (16-byte chunks of 8 bf16
// in, 8-byte chunks of 8 int8 out), fp32 math with IEEE division:
//  * activations (per token): s[m] = max(max_k |x[m][k]|, 1e-5) / 127, q = trunc(x / s + 0.5 sign) (round half away
//    from zero): the reference's _quant_rows, moondream/gpu/tgemm.py:81-91;
//  * weights (per output channel): s[n] = max(max_k |w[n][k]|, 1e-8) / 127, q = clamp(round-half-even(w / s), +-127):
//    HI8Lin.__init__, moondream/gpu/hgemm.py:101-106.
#include "common.h"

namespace {

template <bool WEIGHT>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, long ldx,
                                                         int8_t* __restrict__ q, long ldq, float* __restrict__ s,
                                                         int K) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + (long)m * ldx;
  const int nc = K / 8;
  float amax = 0.f;
  for (int c = tid; c < nc; c += 256) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + c * 8);
#pragma unroll
    for (int e = 0; e < 4; e++) amax = fmaxf(amax, fmaxf(fabsf(lo_bf(v[e])), fabsf(hi_bf(v[e]))));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(amax, WEIGHT ? 1e-8f : 1e-5f) / 127.0f;
  if (tid == 0) s[m] = sc;
  int8_t* qr = q + (long)m * ldq;
  for (int c = tid; c < nc; c += 256) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + c * 8);
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t u = v[e >> 1];
      const float f = (e & 1) ? hi_bf(u) : lo_bf(u);
      const float t = f / sc;
      const int qi = WEIGHT ? (int)fminf(fmaxf(rintf(t), -127.f), 127.f) : (int)(t + (t >= 0.f ? 0.5f : -0.5f));
      w[e >> 2] |= ((uint32_t)qi & 0xffu) << (8 * (e & 3));
    }
    *reinterpret_cast<u32x2*>(qr + c * 8) = u32x2{w[0], w[1]};
  }
}

}  // namespace

extern "C" int mx_quant_rows_i8(hipStream_t st, const uint16_t* x, long ldx, int8_t* q, long ldq, float* s, int M,
                                int K) {
  if (!x || !q || !s) return MX_ENULL;
  if (M < 1 || K < 8 || K % 8 || ldx < K || ldx % 8 || ldq < K || ldq % 8) return MX_ESHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)q & 7)) return MX_ELAYOUT;
  hipLaunchKernelGGL(quant_rows_kernel<false>, dim3(M), dim3(256), 0, st, x, ldx, q, ldq, s, K);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_quant_weight_i8(hipStream_t st, const uint16_t* w, long ldw, int8_t* q, long ldq, float* s, int N,
                                  int K) {
  if (!w || !q || !s) return MX_ENULL;
  if (N < 1 || K < 8 || K % 8 || ldw < K || ldw % 8 || ldq < K || ldq % 8) return MX_ESHAPE;
  if (((uintptr_t)w & 15) || ((uintptr_t)q & 7)) return MX_ELAYOUT;
  hipLaunchKernelGGL(quant_rows_kernel<true>, dim3(N), dim3(256), 0, st, w, ldw, q, ldq, s, K);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
