// Wave-level GEMV helpers shared by the batch-1 decode kernels (decode.hip, decode_mk.hip).
// Layout: a row of K bf16 is K / 8 chunks of 16 bytes; lane l of a 64-wide wave holds chunks l, l + 64, ... of a row
// (1 KB per wave per load instruction), multiplies them with the activation's chunks at the same positions in fp32
// and the row sums are finished by a wave reduction.
#pragma once
#include "common.h"

namespace {

__device__ __forceinline__ float dot8(u32x4 w, u32x4 x, float acc) {
#pragma unroll
  for (int e = 0; e < 4; e++) {
    acc = __builtin_fmaf(lo_bf(w[e]), lo_bf(x[e]), acc);
    acc = __builtin_fmaf(hi_bf(w[e]), hi_bf(x[e]), acc);
  }
  return acc;
}

// LayerNorm of a row held as KC chunks per lane (chunk c = lane + 64 i), with gamma / beta chunks gc / bc loaded by
// the caller (before its weight rows, so the normalisation need not wait for them): bf16 result in place (torch
// F.layer_norm numerics: fp32 statistics, biased variance, one rounding).
// (DPP: the wave sums by wave_total, fewer steps than wave_sum's LDS permutes, another fp32 summation order)
template <int KC, bool DPP = false>
__device__ __forceinline__ void ln_chunks(u32x4 (&xc)[KC], const u32x4 (&gc)[KC], const u32x4 (&bc)[KC], float eps,
                                          int K, int lane) {
  auto red = [](float v) { return DPP ? wave_total(v) : wave_sum(v); };
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < KC; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) s += lo_bf(xc[i][e]) + hi_bf(xc[i][e]);
  const float mean = red(s) / (float)K;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < KC; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float d0 = lo_bf(xc[i][e]) - mean, d1 = hi_bf(xc[i][e]) - mean;
      ss += d0 * d0 + d1 * d1;
    }
  const float rstd = 1.0f / sqrtf(red(ss) / (float)K + eps);
#pragma unroll
  for (int i = 0; i < KC; i++) {
    const u32x4 g = gc[i], b = bc[i];
#pragma unroll
    for (int e = 0; e < 4; e++)
      xc[i][e] = pack2((lo_bf(xc[i][e]) - mean) * rstd * lo_bf(g[e]) + lo_bf(b[e]),
                       (hi_bf(xc[i][e]) - mean) * rstd * hi_bf(g[e]) + hi_bf(b[e]));
  }
}

// Sum R per-lane values over the wave (R a power of two <= 64) with 6 + R - 1 - log2(R) exchanges instead of 6 R:
// each of the first log2(R) exchanges (lane distance 32, 16, ...) halves the values a lane holds (a lane keeps the
// half selected by its lane bit and receives its partner's copy of that half), then a butterfly over the remaining
// lane bits completes the sums. Lane l ends with the total of value l >> (6 - log2 R).
template <int R>
__device__ __forceinline__ float reduce_rows(float (&v)[R], int lane) {
  constexpr int L = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : R == 16 ? 4 : R == 32 ? 5 : 6;
  static_assert((1 << L) == R, "R must be a power of two <= 64");
#pragma unroll
  for (int st = 0; st < L; st++) {
    const int d = 32 >> st, H = R >> (st + 1);
    const bool up = lane & d;
#pragma unroll
    for (int j = 0; j < H; j++) {
      const float keep = up ? v[j + H] : v[j];
      const float send = up ? v[j] : v[j + H];
      v[j] = keep + __shfl_xor(send, d, 64);
    }
  }
  float t = v[0];
#pragma unroll
  for (int d = 32 >> L; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
  return t;
}

template <int KC>
__device__ __forceinline__ void load_vec(u32x4 (&xc)[KC], const uint16_t* x, int lane) {
#pragma unroll
  for (int i = 0; i < KC; i++) xc[i] = *reinterpret_cast<const u32x4*>(x + (lane + 64 * i) * 8);
}

// Argmax key: orderable bits of the bf16 logit in the high word, (0xffffffff - index) in the low word, so the
// largest key is the largest logit and, among equal logits, the smallest index.
__device__ __forceinline__ unsigned long long amax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}

}  // namespace
