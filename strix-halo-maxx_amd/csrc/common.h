// Shared device helpers for the gfx950 (CDNA4) kernels of this library.
// bf16 tensors are passed across the C ABI as uint16_t* (raw bit patterns); every kernel accumulates in fp32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Status codes shared by every entry point (0 = launched).
#define MX_OK 0
#define MX_EBADCFG -1    // unknown tile config / head dim / mode
#define MX_ESHAPE -2     // shape or stride not supported (alignment, divisibility)
#define MX_ESPLIT -3     // split-K workspace too small
#define MX_ELAYOUT -4    // operand layout mismatch
#define MX_ELAUNCH -5    // the HIP launch itself failed
#define MX_ENULL -6      // a required pointer is null

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even (the rounding torch uses for .to(torch.bfloat16)); NaN stays NaN.
// gfx950 does this in hardware (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// round an fp32 value to the nearest bf16 and return it as fp32
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// GELU, tanh form: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), evaluated in fp32 like torch's
// F.gelu(x, approximate="tanh") on a bf16 tensor (upcast, compute, round once). Since 1 + tanh(u) = 2 / (1 + exp(-2u)),
// this is x / (1 + exp(-2u)) with -2u / ln 2 = x (c1 + c2 x^2): one hardware exp2 (v_exp_f32), one reciprocal
// (v_rcp_f32) and five plain operations, and no cancellation in 1 + tanh(u) for negative u. Within a few fp32 ulp of
// the formula; saturates to x for large u (exp2 -> 0) and to -0 for very negative u (exp2 -> inf, rcp -> 0).
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float c1 = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634);  // -2 sqrt(2/pi) / ln 2
  constexpr float c2 = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634 * 0.044715);
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(c2, x * x, c1));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
// GELU, erf form (torch nn.GELU() default): 0.5 x (1 + erf(z)), z = x / sqrt 2, in torch's order, with
// erf(z) = sign(z) (1 - erfc(|z|)) and erfc from the Chebyshev fit of Numerical Recipes (2nd ed., section 6.2, erfcc):
// erfc(a) = t exp(-a^2 + P(t)), t = 1 / (1 + a / 2), P of degree 9, fractional error below 1.2e-7 for every a >= 0.
// One hardware reciprocal and one exp2 like gelu_tanh, against the ~5x costlier library erff. For every bf16 input
// the bf16 result equals that of the same formula with a correctly rounded erf (checked exhaustively in fp32 on the
// CPU, 33,409 inputs in [-12, 12]; beyond, erf rounds to +-1 either way); the hardware rcp / exp2 can move a result
// by one bf16 ulp.
__device__ __forceinline__ float gelu_erf(float x) {
  const float z = x * 0.7071067811865476f;
  const float a = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, a, 1.0f));
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  const float erfc_a = t * __builtin_amdgcn_exp2f((p - a * a) * 1.4426950408889634f);
  const float e = 1.0f - erfc_a;
  return 0.5f * x * (1.0f + (z < 0.0f ? -e : e));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// DPP lane moves (VALU, no LDS round trip): CTRL quad_perm 0x00-0xff, row_mirror 0x140, row_half_mirror 0x141,
// row_bcast15 0x142, row_bcast31 0x143; rows outside ROW_MASK return old.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xf, false));
}
// Sum of v over the 64 lanes, returned wave-uniform: pairs, quads, half rows and rows by DPP butterflies, then rows
// 0 + 1 and 2 + 3 by row_bcast15 and the whole wave into lane 63 by row_bcast31. ~6 VALU steps instead of 6 LDS
// permutes; a fixed order (deterministic), not the xor-butterfly order of wave_sum.
__device__ __forceinline__ float wave_total(float v) {
  v += dpp_mov<0xb1>(0.f, v);        // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4e>(0.f, v);        // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(0.f, v);       // row_half_mirror
  v += dpp_mov<0x140>(0.f, v);       // row_mirror
  v += dpp_mov<0x142, 0xa>(0.f, v);  // row_bcast15 into rows 1, 3
  v += dpp_mov<0x143, 0xc>(0.f, v);  // row_bcast31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Max of v over the 64 lanes, wave-uniform, by the same DPP steps as wave_total (exact in any order; rows a broadcast
// skips keep their own value). Every lane must be active.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v, v));
  v = fmaxf(v, dpp_mov<0x4e>(v, v));
  v = fmaxf(v, dpp_mov<0x141>(v, v));
  v = fmaxf(v, dpp_mov<0x140>(v, v));
  v = fmaxf(v, dpp_mov<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp_mov<0x143, 0xc>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}


__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// 32x32x16 bf16 MFMA (gfx950). Operand lane layout: lane l holds row/col (l & 31) and 8 consecutive k values of
// k-group (l >> 5). Result lane layout: lane l holds column (l & 31); register r holds row 8*(r/4) + 4*(l>>5) + (r%4).
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ---- asynchronous global -> LDS copies (LDS-DMA) and their completion waits
#pragma clang diagnostic ignored "-Winline-asm"

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) void*)p);
}

// 64 lanes x 16 bytes from global (per-lane address) into LDS at m0 = lds (wave-uniform) + 16 * lane. The compiler
// does not see the LDS write: the caller waits for it with wait_vm / wait_stages and a barrier before reading.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// Same copy with a wave-uniform 64-bit base (SGPR pair) and a per-lane 32-bit byte offset.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t bu = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(bu),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most E + min(ahead, A) * LPS loads are still in flight: ring stages of LPS loads each, plus E loads
// issued after the awaited stage's own (in the same issue call).
template <int LPS, int A, int E = 0>
__device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      wait_vm<E + A * LPS>();
      return;
    }
    wait_stages<LPS, A - 1, E>(ahead);
  } else {
    wait_vm<E>();
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
// LDS transpose read (ds_read_b64_tr_b16). Within each 16-lane group, lane j = a + 4 e (a, e in 0..3) supplies the
// address of 4 consecutive bf16 of some row; lane 4 a' + b then receives element b of the reads of lanes
// a', a' + 4, a' + 8, a' + 12 (in that order). With lane a + 4 e pointing at M[r0 + e][c0 + 4 a], every lane j of
// the group receives the column M[r0 .. r0 + 3][c0 + j].
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Combine the two 32-lane halves of a wave (v_permlane32_swap): every lane receives (v[l & 31], v[(l & 31) + 32]),
// so both halves compute the same low-then-high result.
__device__ __forceinline__ float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
