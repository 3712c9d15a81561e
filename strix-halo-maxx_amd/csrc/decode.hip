// Batch-1 greedy decode kernels for the moondream2 text model (hidden 2048, 32 heads x 64, MLP 8192, vocab 51200).
//
// A decode step is HBM-bound: every weight (2.6 GB) is read once per token. The step is 3 kernels per layer plus
// 2 per token, all replayed from one HIP graph, with the step's position and the token living in device memory:
//   ln_gemv2      h = LN(x) (recomputed per wave from the 4 KB row), [qkv | fc1] = h [Wqkv | Wfc1]^T + b, GELU on
//                 the fc1 part (the reference's qkv and fc1 both read the same LN output, md2fast.py:173-198)
//   attn_fc2      rope on q / k of the new token, K/V append at `pos`, attention over keys 0..pos (one workgroup per
//                 head, a one-pass online softmax per wave, the 16 waves merged in LDS) and, on workgroups of their
//                 own in the same launch, y2 = bf16(fc2(g) + b2), which needs only the fc1 output
//   gemv_res2     x' = bf16(y2 + bf16(bf16(proj(a) + bp) + x)): the parallel residual of md2fast.py:198 with the
//                 reference's rounding order
//   (decode_attn + gemv_dual_res: the same two steps as attention alone, then both GEMVs in one pass)
//   ln_gemv_argmax  logits = LN(x) Wlm^T + b (bf16, as the reference's bf16 lm_head) and a per-workgroup argmax
//   embed_step    reduce the per-workgroup argmaxes (first index wins ties, like torch.argmax), append the token to
//                 the output, x = wte[token], advance the position counter
// GEMV layout: a 64-wide wave owns R weight rows; lane l reads 16-byte chunks l, l + 64, ... of each row (1 KB per
// wave per load instruction, all rows' loads issued before any arithmetic), fp32 FMAs, a wave reduction per row.
#include "common.h"
#include "gemv.h"

namespace {

// ---------------------------------------------------------------------------------------------- ln_gemv2
template <int KC, int R>
__global__ __launch_bounds__(256) void ln_gemv2_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
                                                       const uint16_t* __restrict__ beta, float eps,
                                                       const uint16_t* __restrict__ W, long ldw,
                                                       const float* __restrict__ bias, int N, int n1,
                                                       uint16_t* __restrict__ out1, uint16_t* __restrict__ out2,
                                                       int act2) {
  constexpr int SH = 6 - (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);  // lane >> SH = row it finishes
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= N) return;
  const int nme = row0 + (lane >> SH);  // the output row this lane completes
  // the small operands first, so the LayerNorm runs while the weight rows stream in
  u32x4 xc[KC], gc[KC], bc[KC];
  load_vec<KC>(xc, x, lane);
  load_vec<KC>(gc, gamma ? gamma : x, lane);  // x: a stand-in when there is no LayerNorm (not used)
  load_vec<KC>(bc, beta ? beta : x, lane);
  const float bme = (bias && nme < N) ? bias[nme] : 0.f;
  u32x4 wv[R][KC];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint16_t* wr = W + (long)min(row0 + r, N - 1) * ldw;
#pragma unroll
    for (int i = 0; i < KC; i++) wv[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (lane + 64 * i) * 8));
  }
  if (gamma) ln_chunks<KC>(xc, gc, bc, eps, KC * 512, lane);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < KC; i++) acc[r] = dot8(wv[r][i], xc[i], acc[r]);
  }
  const float tot = reduce_rows<R>(acc, lane);
  if ((lane & ((1 << SH) - 1)) == 0 && nme < N) {
    float v = rbf(tot + bme);
    if (nme < n1) {
      out1[nme] = f2bf(v);
    } else {
      if (act2 == 1) v = gelu_tanh(v);
      else if (act2 == 2) v = gelu_erf(v);
      out2[nme - n1] = f2bf(v);
    }
  }
}

// ---------------------------------------------------------------------------------------------- gemv_dual_res
template <int KC1, int KC2, int R>
__global__ __launch_bounds__(256) void gemv_dual_res_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ W2,
                                                            const float* __restrict__ b2,
                                                            const uint16_t* __restrict__ a, const uint16_t* __restrict__ Wp,
                                                            const float* __restrict__ bp,
                                                            const uint16_t* __restrict__ xres, uint16_t* __restrict__ out,
                                                            int N) {
  // 2 R sums per wave (fc2 rows, then proj rows): lane l finishes sum l >> SH; the proj sum of row r sits 32 lanes
  // above its fc2 sum
  constexpr int SH = 6 - (R == 1 ? 1 : R == 2 ? 2 : R == 4 ? 3 : 4);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= N) return;
  const int nme = row0 + ((lane >> SH) & (R - 1));
  u32x4 gc[KC1], ac[KC2];
  load_vec<KC1>(gc, g, lane);
  load_vec<KC2>(ac, a, lane);
  const bool in = nme < N;
  const float b2me = in ? b2[nme] : 0.f, bpme = in ? bp[nme] : 0.f, xme = in ? bf2f(xres[nme]) : 0.f;
  u32x4 w2[R][KC1], wp[R][KC2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);
#pragma unroll
    for (int i = 0; i < KC1; i++)
      w2[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W2 + (long)n * KC1 * 512 + (lane + 64 * i) * 8));
#pragma unroll
    for (int i = 0; i < KC2; i++)
      wp[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Wp + (long)n * KC2 * 512 + (lane + 64 * i) * 8));
  }
  float acc[2 * R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0.f;
    acc[R + r] = 0.f;
#pragma unroll
    for (int i = 0; i < KC1; i++) acc[r] = dot8(w2[r][i], gc[i], acc[r]);
#pragma unroll
    for (int i = 0; i < KC2; i++) acc[R + r] = dot8(wp[r][i], ac[i], acc[R + r]);
  }
  const float tot = reduce_rows<2 * R>(acc, lane);      // lanes < 32: fc2 sums, lanes >= 32: proj sums
  const float sp = __shfl_xor(tot, 32, 64);
  if (lane < 32 && (lane & ((1 << SH) - 1)) == 0 && in) {
    const float pr = rbf(rbf(sp + bpme) + xme);
    out[nme] = f2bf(rbf(tot + b2me) + pr);
  }
}

// ---------------------------------------------------------------------------------------------- W8A8 GEMVs
// The reference's W8A8 text linears (moondream/gpu/hgemm.py:95-137) at batch 1: int8 weight rows (per-row scale sw),
// the activation row quantised per token (s = max(amax, 1e-5) / 127, q = trunc(v + 0.5 sign), tgemm.py:81-91) once
// per workgroup into LDS, int8 dot products (v_dot4) summed exactly in int32, then the fp32 dequant
// ((acc * s) * sw) + b and any GELU on that fp32 value before the one bf16 rounding (i8gemm.hip:181-197).
// Layout: a row of K int8 is K / 16 chunks of 16 bytes; lane l holds chunks l + 64 j (j < KI), i.e. elements
// 16 (l + 64 j) .. +15, and loads the activation values at the same positions (two 8-wide bf16 chunks per int8 chunk).
typedef int i32x4v __attribute__((ext_vector_type(4)));

// Exact int32 sum over the wave of R per-lane values (the reduce_rows exchange pattern); lane l ends with the total of
// value l >> (6 - log2 R).
template <int R>
__device__ __forceinline__ int reduce_rows_i(int (&v)[R], int lane) {
  constexpr int L = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : R == 16 ? 4 : R == 32 ? 5 : 6;
  static_assert((1 << L) == R, "R must be a power of two <= 64");
#pragma unroll
  for (int st = 0; st < L; st++) {
    const int d = 32 >> st, H = R >> (st + 1);
    const bool up = lane & d;
#pragma unroll
    for (int j = 0; j < H; j++) {
      const int keep = up ? v[j + H] : v[j];
      const int send = up ? v[j] : v[j + H];
      v[j] = keep + __shfl_xor(send, d, 64);
    }
  }
  int t = v[0];
#pragma unroll
  for (int d = 32 >> L; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
  return t;
}

// 16 int8 x int8 products of one activation chunk and one weight chunk (4 packed words each), added to acc.
__device__ __forceinline__ int dot16_i8(const i32x4v& a, const u32x4& b, int acc) {
#pragma unroll
  for (int w = 0; w < 4; w++) acc = __builtin_amdgcn_sdot4(a[w], (int)b[w], acc, false);
  return acc;
}

// Workgroup-wide max / sum of one value per thread through red (NW floats, NW = waves per workgroup); every thread
// gets the result.
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < NW; w++) m = fmaxf(m, red[w]);
  return m;
}
__device__ __forceinline__ float block_sum4(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// Per-token int8 quantisation (tgemm.py:81-91 _quant_rows: s = max(max |x|, 1e-5) / 127, q = trunc(x / s + 0.5 sign),
// IEEE division) of a vector of 64 NW E values (thread t holds values t E .. t E + E - 1, already rounded to bf16)
// shared by the 64 NW threads of a workgroup, done once per workgroup: qs receives the int8 values in k order (4 per
// word, the order of a weight row's 16-byte chunks); the scale is the workgroup's (through smax, NW floats). The
// caller synchronises before reading qs.
template <int E, int NW = 4>
__device__ __forceinline__ float quant_vals_block_i8(const float (&f)[E], uint32_t* qs, float* smax) {
  static_assert(E % 4 == 0, "whole words per thread");
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < E; i++) amax = fmaxf(amax, fabsf(f[i]));
  amax = block_max<NW>(amax, smax);
  const float s = fmaxf(amax, 1e-5f) / 127.0f;
#pragma unroll
  for (int i = 0; i < E / 4; i++) {
    uint32_t word = 0u;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const float t = f[4 * i + b] / s;
      const int qi = (int)(t + (t >= 0.f ? 0.5f : -0.5f));
      word |= ((uint32_t)qi & 0xffu) << (8 * b);
    }
    qs[threadIdx.x * (E / 4) + i] = word;
  }
  return s;
}

// This thread's E consecutive bf16 elements of x (t E .. t E + E - 1) as fp32.
template <int E>
__device__ __forceinline__ void load_slice(const uint16_t* __restrict__ x, float (&f)[E]) {
#pragma unroll
  for (int i = 0; i < E / 4; i++) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(x + threadIdx.x * E + 4 * i);
    f[4 * i] = lo_bf(v.x);
    f[4 * i + 1] = hi_bf(v.x);
    f[4 * i + 2] = lo_bf(v.y);
    f[4 * i + 3] = hi_bf(v.y);
  }
}

template <int E, int NW = 4>
__device__ __forceinline__ float quant_block_i8(const uint16_t* __restrict__ x, uint32_t* qs, float* smax) {
  float f[E];
  load_slice<E>(x, f);
  return quant_vals_block_i8<E, NW>(f, qs, smax);
}

// [qkv | fc1] = dequant(quant(LN(x)) . Wq^T); out1 = rows < n1 (bf16), out2 = GELU rows >= n1 (act2 1 tanh, 2 erf).
// The LayerNorm and the quantisation of x run once per workgroup (thread t on elements 4 KI t ..), into LDS, while
// the weight loads are in flight.
template <int KI, int R>
__global__ __launch_bounds__(256) void ln_gemv2_i8_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ gamma,
                                                          const uint16_t* __restrict__ beta, float eps,
                                                          const int8_t* __restrict__ Wq, long ldw,
                                                          const float* __restrict__ sw, const float* __restrict__ bias,
                                                          int N, int n1, uint16_t* __restrict__ out1,
                                                          uint16_t* __restrict__ out2, int act2) {
  constexpr int SH = 6 - (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);
  constexpr int E = 4 * KI;  // elements of x per thread
  __shared__ __attribute__((aligned(16))) uint32_t qs[KI * 256];
  __shared__ float red[3][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const bool active = row0 < N;  // every wave takes part in the workgroup's LayerNorm and quantisation (barriers)
  const int nme = row0 + (lane >> SH);
  float f[E];
  load_slice<E>(x, f);
  const float bme = (bias && active && nme < N) ? bias[nme] : 0.f, swme = active && nme < N ? sw[nme] : 0.f;
  u32x4 wv[R][KI];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int8_t* wr = Wq + (long)min(row0 + r, N - 1) * ldw;
#pragma unroll
    for (int j = 0; j < KI; j++) wv[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (lane + 64 * j) * 16));
  }
  if (gamma) {  // torch F.layer_norm numerics: fp32 statistics, biased variance, one rounding to bf16
    constexpr float K = KI * 1024;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < E; i++) sum += f[i];
    const float mean = block_sum4(sum, red[0]) / K;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < E; i++) ss += (f[i] - mean) * (f[i] - mean);
    const float rstd = 1.0f / sqrtf(block_sum4(ss, red[1]) / K + eps);
#pragma unroll
    for (int i = 0; i < E; i++) {
      const int k = threadIdx.x * E + i;
      f[i] = rbf((f[i] - mean) * rstd * bf2f(gamma[k]) + bf2f(beta[k]));
    }
  }
  const float sx = quant_vals_block_i8<E>(f, qs, red[2]);
  __syncthreads();
  if (!active) return;
  i32x4v q[KI];
#pragma unroll
  for (int j = 0; j < KI; j++) q[j] = *reinterpret_cast<const i32x4v*>(&qs[4 * (lane + 64 * j)]);
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0;
#pragma unroll
    for (int j = 0; j < KI; j++) acc[r] = dot16_i8(q[j], wv[r][j], acc[r]);
  }
  const int tot = reduce_rows_i<R>(acc, lane);
  if ((lane & ((1 << SH) - 1)) == 0 && nme < N) {
    const float t = (float)tot * sx;
    float v = t * swme + bme;
    if (nme < n1) {
      out1[nme] = f2bf(v);
    } else {
      if (act2 == 1) v = gelu_tanh(v);
      else if (act2 == 2) v = gelu_erf(v);
      out2[nme - n1] = f2bf(v);
    }
  }
}

// x' = bf16(bf16(fc2(g)) + bf16(bf16(proj(a)) + x)) with both Linears W8A8 (the parallel residual of
// md2fast.py:198 through lin_res / mlp with fused_res off). g and a are quantised once per workgroup into LDS while
// the weight loads are in flight.
template <int KI1, int KI2, int R>
__global__ __launch_bounds__(256) void gemv_dual_res_i8_kernel(
    const uint16_t* __restrict__ g, const int8_t* __restrict__ W2, const float* __restrict__ sw2,
    const float* __restrict__ b2, const uint16_t* __restrict__ a, const int8_t* __restrict__ Wp,
    const float* __restrict__ swp, const float* __restrict__ bp, const uint16_t* __restrict__ xres,
    uint16_t* __restrict__ out, int N) {
  constexpr int SH = 6 - (R == 1 ? 1 : R == 2 ? 2 : R == 4 ? 3 : 4);
  __shared__ __attribute__((aligned(16))) uint32_t qgs[KI1 * 256], qas[KI2 * 256];
  __shared__ float smax[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const bool active = row0 < N;  // every wave takes part in the workgroup's quantisation (barriers)
  const int nme = row0 + ((lane >> SH) & (R - 1));
  const bool in = active && nme < N;
  u32x4 w2[R][KI1], wp[R][KI2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);
#pragma unroll
    for (int j = 0; j < KI1; j++)
      w2[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W2 + (long)n * KI1 * 1024 + (lane + 64 * j) * 16));
#pragma unroll
    for (int j = 0; j < KI2; j++)
      wp[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Wp + (long)n * KI2 * 1024 + (lane + 64 * j) * 16));
  }
  const float b2me = in ? b2[nme] : 0.f, bpme = in ? bp[nme] : 0.f, xme = in ? bf2f(xres[nme]) : 0.f;
  const float sw2me = in ? sw2[nme] : 0.f, swpme = in ? swp[nme] : 0.f;
  const float sg = quant_block_i8<KI1 * 4>(g, qgs, smax[0]);
  const float sa = quant_block_i8<KI2 * 4>(a, qas, smax[1]);
  __syncthreads();
  if (!active) return;
  i32x4v qg[KI1], qa[KI2];
#pragma unroll
  for (int j = 0; j < KI1; j++) qg[j] = *reinterpret_cast<const i32x4v*>(&qgs[4 * (lane + 64 * j)]);
#pragma unroll
  for (int j = 0; j < KI2; j++) qa[j] = *reinterpret_cast<const i32x4v*>(&qas[4 * (lane + 64 * j)]);
  int acc[2 * R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0;
    acc[R + r] = 0;
#pragma unroll
    for (int j = 0; j < KI1; j++) acc[r] = dot16_i8(qg[j], w2[r][j], acc[r]);
#pragma unroll
    for (int j = 0; j < KI2; j++) acc[R + r] = dot16_i8(qa[j], wp[r][j], acc[R + r]);
  }
  const int tot = reduce_rows_i<2 * R>(acc, lane);  // lanes < 32: fc2 sums, lanes >= 32: proj sums
  const int sp = __shfl_xor(tot, 32, 64);
  if (lane < 32 && (lane & ((1 << SH) - 1)) == 0 && in) {
    const float tf = (float)tot * sg, tp = (float)sp * sa;
    const float vf = tf * sw2me + b2me, vp = tp * swpme + bpme;
    out[nme] = f2bf(rbf(vf) + rbf(rbf(vp) + xme));
  }
}

// ---------------------------------------------------------------------------------------------- lm head + argmax
template <int KC, int R>
__global__ __launch_bounds__(256) void ln_gemv_argmax_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gamma,
                                                             const uint16_t* __restrict__ beta, float eps,
                                                             const uint16_t* __restrict__ W, long ldw,
                                                             const float* __restrict__ bias, int N,
                                                             uint16_t* __restrict__ logits,
                                                             unsigned long long* __restrict__ part) {
  constexpr int SH = 6 - (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);
  __shared__ unsigned long long sbest[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  unsigned long long best = 0ull;
  if (row0 < N) {
    const int nme = row0 + (lane >> SH);
    u32x4 xc[KC], gc[KC], bc[KC];
    load_vec<KC>(xc, x, lane);
    load_vec<KC>(gc, gamma, lane);
    load_vec<KC>(bc, beta, lane);
    const float bme = nme < N ? bias[nme] : 0.f;
    u32x4 wv[R][KC];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint16_t* wr = W + (long)min(row0 + r, N - 1) * ldw;
#pragma unroll
      for (int i = 0; i < KC; i++) wv[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (lane + 64 * i) * 8));
    }
    ln_chunks<KC>(xc, gc, bc, eps, KC * 512, lane);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      acc[r] = 0.f;
#pragma unroll
      for (int i = 0; i < KC; i++) acc[r] = dot8(wv[r][i], xc[i], acc[r]);
    }
    const float tot = reduce_rows<R>(acc, lane);
    if (nme < N) {
      const float v = rbf(tot + bme);
      if (logits && (lane & ((1 << SH) - 1)) == 0) logits[nme] = f2bf(v);
      best = amax_key(v, nme);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const unsigned long long t = __shfl_xor(best, o, 64);
      best = t > best ? t : best;
    }
  }
  if (lane == 0) sbest[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = sbest[0];
#pragma unroll
    for (int w = 1; w < 4; w++) b = sbest[w] > b ? sbest[w] : b;
    part[blockIdx.x] = b;
  }
}

// ---------------------------------------------------------------------------------------------- embed_step
// state[0] = step s (tokens emitted so far), state[1] = position of the token fed this step (= pos_base + s).
// cap: the number of steps the caches and tokens[] have room for; at s >= cap nothing is recorded and the state stops
// advancing (the host refuses such steps; this keeps a step it did not refuse inside the buffers).
__global__ __launch_bounds__(1024) void embed_step_kernel(const unsigned long long* __restrict__ part, int nparts,
                                                          const uint16_t* __restrict__ wte, int D,
                                                          int* __restrict__ state, int pos_base,
                                                          int* __restrict__ tokens, int cap,
                                                          uint16_t* __restrict__ x) {
  __shared__ unsigned long long sb[16];
  __shared__ int stok;
  unsigned long long b = 0ull;
  for (int i = threadIdx.x; i < nparts; i += 1024) b = part[i] > b ? part[i] : b;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned long long t = __shfl_xor(b, o, 64);
    b = t > b ? t : b;
  }
  if ((threadIdx.x & 63) == 0) sb[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = sb[0];
    for (int w = 1; w < 16; w++) m = sb[w] > m ? sb[w] : m;
    const int tok = (int)(0xffffffffu - (uint32_t)(m & 0xffffffffull));
    stok = tok;
    const int s = state[0];
    if (s < cap) {
      tokens[s] = tok;
      state[1] = pos_base + s;
      state[0] = s + 1;
    }
  }
  __syncthreads();
  const int tok = stok;
  for (int i = threadIdx.x; i < D / 8; i += 1024)
    *reinterpret_cast<u32x4*>(x + i * 8) = *reinterpret_cast<const u32x4*>(wte + (long)tok * D + i * 8);
}

// ---------------------------------------------------------------------------------------------- decode attention
constexpr int DA_W = 16;       // waves per head (one 1024-thread workgroup per head)
constexpr int DA_UNROLL = 8;   // key rounds (8 keys per wave each) whose K and V loads are issued together

// One workgroup per head. Wave w takes keys w * 8 + (lane >> 3) + 128 r, 8 lanes per key (lane & 7 -> dims
// 8 (lane & 7) .. +7), and runs an online softmax over them in one pass: the K and V rows of DA_UNROLL rounds are
// loaded together, scores reduced within each 8-lane group, the wave's running max raised (and its O, l rescaled)
// per batch. The 16 waves' (m, l, O) are merged in LDS. P is rounded to bf16 and l sums the rounded values.
// The body for head h, run by a 1024-thread workgroup (every thread reaches its barriers). With S > 1 the head's
// keys are split over S workgroups: split sp takes keys [sp c, sp c + c) (c = ceil(L / S) rounded up to 8) and writes
// the unnormalised record (M, Lsum, acc[64]) of its 16 waves to part + (h S + sp) 66 for merge_attn; with S = 1 the
// workgroup writes the head's output.
__device__ __forceinline__ void attn_head(int h, int sp, int S, const uint16_t* __restrict__ qkv,
                                          const float* __restrict__ cs, uint16_t* __restrict__ kc,
                                          uint16_t* __restrict__ vc, int H, int ctx, const int* __restrict__ state,
                                          float scale_log2, uint16_t* __restrict__ out, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t qs[64], knew[64], vnew[64];  // bf16 q, k, v of the new token
  __shared__ float rec[DA_W][66];  // (m, l, o[64]) of each wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // state[1] reaches ctx only for a step the host refuses (the embed step's cap); never address past the cache
  const int pos = min(max(state[1], 0), ctx - 1);
  const int L = pos + 1;
  const int chunk = S == 1 ? L : (((L + S - 1) / S + 7) & ~7);
  const int kb = sp * chunk, ke = min(L, kb + chunk);  // this workgroup's keys (empty when kb >= L)
  // the rope's inputs through pointers the compiler cannot see through: loads from the read-only arguments could
  // otherwise be moved freely, behind the cache rows' loads below
  typedef __attribute__((address_space(1))) const float gfloat;
  typedef __attribute__((address_space(1))) const uint16_t gu16;
  const float* cpg = cs + (long)pos * 32;
  const uint16_t* srcg = qkv + h * 64;
  asm volatile("" : "+s"(cpg), "+s"(srcg));
  gfloat* cp = (gfloat*)cpg;
  gu16* src = (gu16*)srcg;
  gu16* ksrc = src + H * 64;
  gu16* vsrc = src + 2 * H * 64;
  const uint16_t* kh = kc + (long)h * ctx * 64;
  const uint16_t* vh = vc + (long)h * ctx * 64;
  // Every wave computes the rope of q and k for the new token (lane d on dim d; fp32, as the prefill rope kernel) from
  // loads issued before the first pass's K / V rows, so that the waits for them do not wait for the cache rows
  // (loads complete in issue order); wave 0 publishes the results.
  const int d = lane, jr = (d & 31) >> 1;
  const float cr = cp[2 * jr], sr = cp[2 * jr + 1];
  const int d0 = d < 32 ? jr : d;
  const uint16_t q0 = src[d0], q1 = src[16 + jr], k0 = ksrc[d0], k1 = ksrc[16 + jr], vn = vsrc[d];
  const int sub = lane & 7, kg = lane >> 3;
  u32x4 kk[DA_UNROLL], vv[DA_UNROLL];
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // K / V rows of one pass, loaded unconditionally (keys past L read row L - 1, so the wait counts stay exact); in the
  // loop, keys past L become zeros (their scores are masked, and 0 * V stays finite) and the row at pos the new
  // token's
  auto load_pass = [&](int b0) {
#pragma unroll
    for (int u = 0; u < DA_UNROLL; u++) {
      const int key = min(b0 + kg + 8 * DA_W * u, L - 1);
      const unsigned off = (unsigned)key * 64u + (unsigned)sub * 8u;  // 32-bit offset from the head's base
      kk[u] = *reinterpret_cast<const u32x4*>(kh + off);
      vv[u] = *reinterpret_cast<const u32x4*>(vh + off);
    }
  };
  asm volatile("" ::: "memory");  // the rope's loads are issued first (no load moves across)
  __builtin_amdgcn_sched_barrier(0);
  load_pass(kb + wave * 8);
  {
    // branch-free (a branch would let the compiler sink these loads behind the cache rows')
    const float qa = bf2f(q0), qb = bf2f(q1), ka = bf2f(k0), kb = bf2f(k1);
    const float qo = __fadd_rn(__fmul_rn(qa, sr), __fmul_rn(qb, cr)), qe = __fsub_rn(__fmul_rn(qa, cr), __fmul_rn(qb, sr));
    const float ko = __fadd_rn(__fmul_rn(ka, sr), __fmul_rn(kb, cr)), ke = __fsub_rn(__fmul_rn(ka, cr), __fmul_rn(kb, sr));
    const float qv = d < 32 ? ((d & 1) ? qo : qe) : qa;
    const float kv = d < 32 ? ((d & 1) ? ko : ke) : ka;
    if (wave == 0) {
      qs[d] = f2bf(qv);
      knew[d] = f2bf(kv);
      vnew[d] = vn;
      if (sp == 0) {  // append the new token's K / V to the cache (this step takes them from LDS)
        kc[((long)h * ctx + pos) * 64 + d] = f2bf(kv);
        vc[((long)h * ctx + pos) * 64 + d] = vn;
      }
    }
  }
  __syncthreads();
  const u32x4 qp = *reinterpret_cast<const u32x4*>(&qs[sub * 8]);  // q dims 8 sub .. +7, bf16 pairs
  float m_run = -1e30f, l_run = 0.f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // the loop bound is wave-uniform (every lane takes part in the wave-wide max); keys past ke are masked
  for (int b0 = kb + wave * 8; b0 < ke; b0 += 8 * DA_W * DA_UNROLL) {
    if (b0 != kb + wave * 8) load_pass(b0);
    const int base = b0 + kg;
#pragma unroll
    for (int u = 0; u < DA_UNROLL; u++)
      if (base + 8 * DA_W * u >= min(pos, ke)) {
        const bool me = base + 8 * DA_W * u == pos && pos < ke;
        kk[u] = me ? *reinterpret_cast<const u32x4*>(&knew[sub * 8]) : zero4;
        vv[u] = me ? *reinterpret_cast<const u32x4*>(&vnew[sub * 8]) : zero4;
      }
    float sv[DA_UNROLL];
    float mb = -1e30f;
#pragma unroll
    for (int u = 0; u < DA_UNROLL; u++) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        s = __builtin_fmaf(lo_bf(kk[u][e]), lo_bf(qp[e]), s);
        s = __builtin_fmaf(hi_bf(kk[u][e]), hi_bf(qp[e]), s);
      }
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 4, 64);
      s = (base + 8 * DA_W * u < ke) ? s * scale_log2 : -INFINITY;
      sv[u] = s;
      mb = fmaxf(mb, s);
    }
    mb = wave_max(mb);
    if (mb > m_run) {  // wave-uniform
      const float alpha = __builtin_amdgcn_exp2f(m_run - mb);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] *= alpha;
      m_run = mb;
    }
#pragma unroll
    for (int u = 0; u < DA_UNROLL; u++) {
      const float p = rbf(__builtin_amdgcn_exp2f(sv[u] - m_run));
      if (sub == 0) l_run += p;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        o[2 * e] = __builtin_fmaf(p, lo_bf(vv[u][e]), o[2 * e]);
        o[2 * e + 1] = __builtin_fmaf(p, hi_bf(vv[u][e]), o[2 * e + 1]);
      }
    }
  }
  // reduce over the 8 key groups of the wave
#pragma unroll
  for (int e = 0; e < 8; e++) {
    o[e] += __shfl_xor(o[e], 8, 64);
    o[e] += __shfl_xor(o[e], 16, 64);
    o[e] += __shfl_xor(o[e], 32, 64);
  }
  l_run = wave_sum(l_run);
  if (kg == 0) {
#pragma unroll
    for (int e = 0; e < 8; e++) rec[wave][2 + sub * 8 + e] = o[e];
  }
  if (lane == 0) { rec[wave][0] = m_run; rec[wave][1] = l_run; }
  __syncthreads();
  // ---- merge the waves: out = sum_w o_w 2^(m_w - M) / sum_w l_w 2^(m_w - M)
  if (tid < 64) {
    float M = -1e30f;
#pragma unroll
    for (int w = 0; w < DA_W; w++) M = fmaxf(M, rec[w][0]);
    float Lt = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < DA_W; w++) {
      const float f = __builtin_amdgcn_exp2f(rec[w][0] - M);
      Lt += rec[w][1] * f;
      acc += rec[w][2 + tid] * f;
    }
    if (S == 1) {
      out[h * 64 + tid] = f2bf(acc / Lt);
    } else {
      float* r = part + ((long)h * S + sp) * 66;
      r[2 + tid] = acc;
      if (tid == 0) { r[0] = M; r[1] = Lt; }
    }
  }
}

// The attention output a[c .. c + E - 1] (within one head) from the S split records of its head:
// bf16(sum_s acc_s 2^(M_s - M) / sum_s Lsum_s 2^(M_s - M)), M = max_s M_s (an empty split has Lsum = acc = 0).
template <int E>
__device__ __forceinline__ void merge_attn(const float* __restrict__ part, int S, int c, float (&f)[E]) {
  const float* r = part + (long)(c >> 6) * S * 66;
  const int d0 = c & 63;
  float M = -1e30f;
  for (int s = 0; s < S; s++) M = fmaxf(M, r[s * 66]);
  float Lt = 0.f, acc[E];
#pragma unroll
  for (int e = 0; e < E; e++) acc[e] = 0.f;
  for (int s = 0; s < S; s++) {
    const float w = __builtin_amdgcn_exp2f(r[s * 66] - M);
    Lt += r[s * 66 + 1] * w;
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] += r[s * 66 + 2 + d0 + e] * w;
  }
#pragma unroll
  for (int e = 0; e < E; e++) f[e] = rbf(acc[e] / Lt);
}

__global__ __launch_bounds__(1024) void decode_attn_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ cs,
                                                           uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                           int H, int ctx, const int* __restrict__ state,
                                                           float scale_log2, uint16_t* __restrict__ out) {
  attn_head(blockIdx.x, 0, 1, qkv, cs, kc, vc, H, ctx, state, scale_log2, out, nullptr);
}

// ---------------------------------------------------------------------------------------------- attention + fc2
// The parallel residual's fc2 GEMV needs only the fc1 output, not the attention's, so it shares the attention's
// launch: workgroups 0 .. H-1 run the attention (one head each, latency-bound on H CUs), workgroups H .. stream the
// fc2 rows on the other CUs, one row per wave, the activation g staged in LDS while the weight row is in flight.
// y2 = bf16(g W2^T + b2), the first rounded term of the residual sum; proj + residual follow in gemv_res2.
template <int KC1>
__global__ __launch_bounds__(1024) void attn_fc2_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ cs,
                                                        uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int H,
                                                        int ctx, const int* __restrict__ state, float scale_log2,
                                                        int S, float* __restrict__ part,
                                                        uint16_t* __restrict__ attn_out, const uint16_t* __restrict__ g,
                                                        const uint16_t* __restrict__ W2, const float* __restrict__ b2,
                                                        uint16_t* __restrict__ y2, int N) {
  if ((int)blockIdx.x < H * S) {
    attn_head(blockIdx.x / S, blockIdx.x % S, S, qkv, cs, kc, vc, H, ctx, state, scale_log2, attn_out, part);
    return;
  }
  __shared__ __attribute__((aligned(16))) uint16_t gs[KC1 * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = ((int)blockIdx.x - H * S) * DA_W + wave;
  const int nr = min(n, N - 1);
  u32x4 w[KC1];
#pragma unroll
  for (int i = 0; i < KC1; i++)
    w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W2 + (long)nr * KC1 * 512 + (lane + 64 * i) * 8));
  const float bn = b2[nr];
  for (int c = threadIdx.x; c < KC1 * 64; c += 64 * DA_W)
    *reinterpret_cast<u32x4*>(&gs[c * 8]) = *reinterpret_cast<const u32x4*>(g + c * 8);
  __syncthreads();
  if (n >= N) return;
  float acc[1] = {0.f};
#pragma unroll
  for (int i = 0; i < KC1; i++) acc[0] = dot8(w[i], *reinterpret_cast<const u32x4*>(&gs[(lane + 64 * i) * 8]), acc[0]);
  const float tot = reduce_rows<1>(acc, lane);
  if (lane == 0) y2[n] = f2bf(tot + bn);
}

// The W8A8 form: g quantised per token once per fc2 workgroup (16 waves) into LDS, int8 dots summed exactly,
// y2 = bf16(((acc s_g) s_w) + b2) (the epilogue of the W8A8 dual GEMV). Its 16.8 MB of int8 rows stream in less time
// than the attention takes, so the fc2 workgroups start FC2_I8_NAP x 1024 cycles late: the attention's cache loads
// then do not queue behind them (decode 1762 -> 1815 tok/s at 4; the bf16 form, whose 33.5 MB take as long as the
// attention, only loses from a delay).
constexpr int FC2_I8_NAP = 4;
template <int KI1>
__global__ __launch_bounds__(1024) void attn_fc2_i8_kernel(const uint16_t* __restrict__ qkv,
                                                           const float* __restrict__ cs, uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vc, int H, int ctx,
                                                           const int* __restrict__ state, float scale_log2, int S,
                                                           float* __restrict__ part, uint16_t* __restrict__ attn_out,
                                                           const uint16_t* __restrict__ g,
                                                           const int8_t* __restrict__ W2, const float* __restrict__ sw2,
                                                           const float* __restrict__ b2, uint16_t* __restrict__ y2,
                                                           int N) {
  if ((int)blockIdx.x < H * S) {
    attn_head(blockIdx.x / S, blockIdx.x % S, S, qkv, cs, kc, vc, H, ctx, state, scale_log2, attn_out, part);
    return;
  }
  __shared__ __attribute__((aligned(16))) uint32_t qgs[KI1 * 256];
  __shared__ float smax[DA_W];
#pragma unroll
  for (int i = 0; i < FC2_I8_NAP; i++) __builtin_amdgcn_s_sleep(16);  // 16 x 64 cycles each
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = ((int)blockIdx.x - H * S) * DA_W + wave;
  const int nr = min(n, N - 1);
  u32x4 w[KI1];
#pragma unroll
  for (int j = 0; j < KI1; j++)
    w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W2 + (long)nr * KI1 * 1024 + (lane + 64 * j) * 16));
  const float swn = sw2[nr], bn = b2[nr];
  // K2 = 1024 KI1 values over 1024 threads: KI1 per thread
  const float sg = quant_block_i8<KI1, DA_W>(g, qgs, smax);
  __syncthreads();
  if (n >= N) return;
  int acc[1] = {0};
#pragma unroll
  for (int j = 0; j < KI1; j++)
    acc[0] = dot16_i8(*reinterpret_cast<const i32x4v*>(&qgs[4 * (lane + 64 * j)]), w[j], acc[0]);
  const int tot = reduce_rows_i<1>(acc, lane);
  if (lane == 0) {
    const float tf = (float)tot * sg;
    const float vf = tf * swn + bn;
    y2[n] = f2bf(vf);
  }
}

// ---------------------------------------------------------------------------------------------- gemv_res2
// x' = bf16(y2 + bf16(bf16(proj(a) + bp) + x)): the rest of the parallel residual after attn_fc2 (the same
// roundings, in the same order, as gemv_dual_res). R rows per wave, 4 waves per workgroup. S > 1: a is merged from
// the attention's split records into LDS first (while the weight rows are in flight).
template <int KC2, int R>
__global__ __launch_bounds__(256) void gemv_res2_kernel(const uint16_t* __restrict__ y2, const uint16_t* __restrict__ a,
                                                        int S, const float* __restrict__ part,
                                                        const uint16_t* __restrict__ Wp, const float* __restrict__ bp,
                                                        const uint16_t* __restrict__ xres, uint16_t* __restrict__ out,
                                                        int N) {
  constexpr int SH = 6 - (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);
  __shared__ __attribute__((aligned(16))) uint16_t as[KC2 * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const int nme = row0 + (lane >> SH);
  const bool in = row0 < N && nme < N;
  u32x4 wp[R][KC2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);
#pragma unroll
    for (int i = 0; i < KC2; i++)
      wp[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Wp + (long)n * KC2 * 512 + (lane + 64 * i) * 8));
  }
  const float bpme = in ? bp[nme] : 0.f, xme = in ? bf2f(xres[nme]) : 0.f, yme = in ? bf2f(y2[nme]) : 0.f;
  u32x4 ac[KC2];
  if (S > 1) {  // workgroup-uniform
    for (int c = threadIdx.x; c < KC2 * 64; c += 256) {
      float f[8];
      merge_attn<8>(part, S, c * 8, f);
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = pack2(f[2 * e], f[2 * e + 1]);
      *reinterpret_cast<u32x4*>(&as[c * 8]) = v;
    }
    __syncthreads();
    if (row0 >= N) return;
    load_vec<KC2>(ac, as, lane);
  } else {
    if (row0 >= N) return;
    load_vec<KC2>(ac, a, lane);
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < KC2; i++) acc[r] = dot8(wp[r][i], ac[i], acc[r]);
  }
  const float tot = reduce_rows<R>(acc, lane);
  if ((lane & ((1 << SH) - 1)) == 0 && in) out[nme] = f2bf(yme + rbf(rbf(tot + bpme) + xme));
}

// The W8A8 form: a quantised once per workgroup into LDS (the W8A8 dual GEMV's proj half).
template <int KI2, int R>
__global__ __launch_bounds__(256) void gemv_res2_i8_kernel(const uint16_t* __restrict__ y2,
                                                           const uint16_t* __restrict__ a, int S,
                                                           const float* __restrict__ part,
                                                           const int8_t* __restrict__ Wp, const float* __restrict__ swp,
                                                           const float* __restrict__ bp,
                                                           const uint16_t* __restrict__ xres,
                                                           uint16_t* __restrict__ out, int N) {
  constexpr int SH = 6 - (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);
  __shared__ __attribute__((aligned(16))) uint32_t qas[KI2 * 256];
  __shared__ float smax[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const bool active = row0 < N;  // every wave takes part in the workgroup's quantisation (barriers)
  const int nme = row0 + (lane >> SH);
  const bool in = active && nme < N;
  u32x4 wp[R][KI2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);
#pragma unroll
    for (int j = 0; j < KI2; j++)
      wp[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Wp + (long)n * KI2 * 1024 + (lane + 64 * j) * 16));
  }
  const float bpme = in ? bp[nme] : 0.f, swpme = in ? swp[nme] : 0.f;
  const float xme = in ? bf2f(xres[nme]) : 0.f, yme = in ? bf2f(y2[nme]) : 0.f;
  float sa;
  if (S > 1) {  // workgroup-uniform: this thread's KI2 * 4 values of a merged from the split records
    float f[KI2 * 4];
    merge_attn<KI2 * 4>(part, S, threadIdx.x * KI2 * 4, f);
    sa = quant_vals_block_i8<KI2 * 4>(f, qas, smax);
  } else {
    sa = quant_block_i8<KI2 * 4>(a, qas, smax);
  }
  __syncthreads();
  if (!active) return;
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0;
#pragma unroll
    for (int j = 0; j < KI2; j++)
      acc[r] = dot16_i8(*reinterpret_cast<const i32x4v*>(&qas[4 * (lane + 64 * j)]), wp[r][j], acc[r]);
  }
  const int tot = reduce_rows_i<R>(acc, lane);
  if ((lane & ((1 << SH) - 1)) == 0 && in) {
    const float tp = (float)tot * sa;
    const float vp = tp * swpme + bpme;
    out[nme] = f2bf(yme + rbf(rbf(vp) + xme));
  }
}

}  // namespace

extern "C" int mx_ln_gemv2(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta, float eps,
                           const uint16_t* W, long ldw, const float* bias, int N, int K, int n1, uint16_t* out1,
                           uint16_t* out2, int act2) {
  if (!x || !W || !out1 || (n1 < N && !out2)) return MX_ENULL;
  if ((gamma == nullptr) != (beta == nullptr)) return MX_ENULL;
  if (N < 1 || n1 < 0 || n1 > N || ldw < K || ldw % 8 || act2 < 0 || act2 > 2) return MX_ESHAPE;
  if (((uintptr_t)x | (uintptr_t)W) & 15) return MX_ELAYOUT;
  constexpr int R = 8;
  const dim3 g((N + 4 * R - 1) / (4 * R));
  if (K == 2048) hipLaunchKernelGGL((ln_gemv2_kernel<4, R>), g, dim3(256), 0, st, x, gamma, beta, eps, W, ldw, bias, N, n1, out1, out2, act2);
  else if (K == 1024) hipLaunchKernelGGL((ln_gemv2_kernel<2, R>), g, dim3(256), 0, st, x, gamma, beta, eps, W, ldw, bias, N, n1, out1, out2, act2);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_gemv_dual_res(hipStream_t st, const uint16_t* g, const uint16_t* W2, const float* b2, int K2,
                                const uint16_t* a, const uint16_t* Wp, const float* bp, int Kp, const uint16_t* xres,
                                uint16_t* out, int N) {
  if (!g || !W2 || !b2 || !a || !Wp || !bp || !xres || !out) return MX_ENULL;
  if (N < 1) return MX_ESHAPE;
  if (((uintptr_t)g | (uintptr_t)W2 | (uintptr_t)a | (uintptr_t)Wp) & 15) return MX_ELAYOUT;
  constexpr int R = 2;
  const dim3 gr((N + 4 * R - 1) / (4 * R));
  if (K2 == 8192 && Kp == 2048)
    hipLaunchKernelGGL((gemv_dual_res_kernel<16, 4, R>), gr, dim3(256), 0, st, g, W2, b2, a, Wp, bp, xres, out, N);
  else if (K2 == 4096 && Kp == 1024)
    hipLaunchKernelGGL((gemv_dual_res_kernel<8, 2, R>), gr, dim3(256), 0, st, g, W2, b2, a, Wp, bp, xres, out, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_lm_argmax_nparts(int N) { return (N + 4 * 8 - 1) / (4 * 8); }

extern "C" int mx_ln_gemv_argmax(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                                 float eps, const uint16_t* W, long ldw, const float* bias, int N, int K,
                                 uint16_t* logits, unsigned long long* part, int nparts) {
  if (!x || !gamma || !beta || !W || !bias || !part) return MX_ENULL;
  if (N < 1 || ldw < K || ldw % 8) return MX_ESHAPE;
  if (nparts < mx_lm_argmax_nparts(N)) return MX_ESPLIT;
  if (((uintptr_t)x | (uintptr_t)W) & 15) return MX_ELAYOUT;
  constexpr int R = 8;
  const dim3 g(mx_lm_argmax_nparts(N));
  if (K == 2048) hipLaunchKernelGGL((ln_gemv_argmax_kernel<4, R>), g, dim3(256), 0, st, x, gamma, beta, eps, W, ldw, bias, N, logits, part);
  else if (K == 1024) hipLaunchKernelGGL((ln_gemv_argmax_kernel<2, R>), g, dim3(256), 0, st, x, gamma, beta, eps, W, ldw, bias, N, logits, part);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_embed_step(hipStream_t st, const unsigned long long* part, int nparts, const uint16_t* wte, int D,
                             int* state, int pos_base, int* tokens, int cap, uint16_t* x) {
  if (!part || !wte || !state || !tokens || !x) return MX_ENULL;
  if (nparts < 1 || D % 8 || cap < 1 || pos_base < 0) return MX_ESHAPE;
  hipLaunchKernelGGL(embed_step_kernel, dim3(1), dim3(1024), 0, st, part, nparts, wte, D, state, pos_base, tokens, cap,
                     x);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// One launch, one 1024-thread workgroup per head: every key of the context is covered by the 16 waves' loads of one
// pass (contexts up to 16 x 8 x 8 = 1024 keys per pass, more in further passes), merged in LDS. S, ws and cnt are
// unused (a split-KV form across workgroups measured no faster) and kept for ABI stability; ws / cnt may be null.
extern "C" int mx_decode_attn(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc, int H,
                              int ctx, const int* state, int S, float scale, float* ws, int* cnt, uint16_t* out) {
  (void)S;
  (void)ws;
  (void)cnt;
  if (!qkv || !cs || !kc || !vc || !state || !out) return MX_ENULL;
  if (H < 1 || ctx < 1) return MX_ESHAPE;
  hipLaunchKernelGGL(decode_attn_kernel, dim3(H), dim3(64 * DA_W), 0, st, qkv, cs, kc, vc, H, ctx, state,
                     scale * 1.4426950408889634f, out);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Attention (as mx_decode_attn) and y2 = bf16(g W2^T + b2) in one launch: H S attention workgroups (S splits of
// each head's keys, 1 <= S <= 8) plus one workgroup per 16 fc2 rows. S = 1 writes attn_out; S > 1 writes the split
// records to part (H S 66 floats) instead, for mx_gemv_res2 to merge. W2 is (N, K2) row-major; K2 = 8192 or 4096.
static int attn_fc2_check(const void* qkv, const void* cs, const void* kc, const void* vc, const void* state, int H,
                          int ctx, int S, const void* part, const void* attn_out, const void* g, const void* W2,
                          const void* b2, const void* y2, int N) {
  if (!qkv || !cs || !kc || !vc || !state || !g || !W2 || !b2 || !y2) return MX_ENULL;
  if (H < 1 || ctx < 1 || N < 1 || S < 1 || S > 8) return MX_ESHAPE;
  if (S == 1 ? !attn_out : !part) return MX_ENULL;
  if (((uintptr_t)g | (uintptr_t)W2) & 15) return MX_ELAYOUT;
  return MX_OK;
}

extern "C" int mx_decode_attn_fc2(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc,
                                  int H, int ctx, const int* state, float scale, int S, float* part,
                                  uint16_t* attn_out, const uint16_t* g, const uint16_t* W2, const float* b2, int K2,
                                  uint16_t* y2, int N) {
  const int rc = attn_fc2_check(qkv, cs, kc, vc, state, H, ctx, S, part, attn_out, g, W2, b2, y2, N);
  if (rc != MX_OK) return rc;
  const dim3 gr(H * S + (N + DA_W - 1) / DA_W);
  const float sl2 = scale * 1.4426950408889634f;
  if (K2 == 8192)
    hipLaunchKernelGGL((attn_fc2_kernel<16>), gr, dim3(64 * DA_W), 0, st, qkv, cs, kc, vc, H, ctx, state, sl2, S, part, attn_out, g, W2, b2, y2, N);
  else if (K2 == 4096)
    hipLaunchKernelGGL((attn_fc2_kernel<8>), gr, dim3(64 * DA_W), 0, st, qkv, cs, kc, vc, H, ctx, state, sl2, S, part, attn_out, g, W2, b2, y2, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// out = bf16(y2 + bf16(bf16(a Wp^T + bp) + xres)); a is the attention output (S = 1) or merged from the S split
// records in part; Wp (N, Kp) row-major, Kp = 2048 or 1024 (= 64 H). out may alias xres.
static int res2_check(const void* y2, const void* a, int S, const void* part, const void* Wp, const void* bp,
                      const void* xres, const void* out, int N) {
  if (!y2 || !Wp || !bp || !xres || !out) return MX_ENULL;
  if (N < 1 || S < 1 || S > 8) return MX_ESHAPE;
  if (S == 1 ? !a : !part) return MX_ENULL;
  if (((uintptr_t)a | (uintptr_t)Wp) & 15) return MX_ELAYOUT;
  return MX_OK;
}

extern "C" int mx_gemv_res2(hipStream_t st, const uint16_t* y2, const uint16_t* a, int S, const float* part,
                            const uint16_t* Wp, const float* bp, int Kp, const uint16_t* xres, uint16_t* out, int N) {
  const int rc = res2_check(y2, a, S, part, Wp, bp, xres, out, N);
  if (rc != MX_OK) return rc;
  constexpr int R = 2;
  const dim3 gr((N + 4 * R - 1) / (4 * R));
  if (Kp == 2048) hipLaunchKernelGGL((gemv_res2_kernel<4, R>), gr, dim3(256), 0, st, y2, a, S, part, Wp, bp, xres, out, N);
  else if (Kp == 1024) hipLaunchKernelGGL((gemv_res2_kernel<2, R>), gr, dim3(256), 0, st, y2, a, S, part, Wp, bp, xres, out, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// W8A8 [qkv | fc1] GEMV with the LayerNorm fused (gamma = beta = null: none): the LN output is quantised per token,
// Wq int8 (N, ldw bytes), sw / bias fp32 per row. K = 2048 or 1024. Replaces HI8Lin on the shared quantised LN output
// (md2fast.py:174-198) for one token.
extern "C" int mx_ln_gemv2_i8(hipStream_t st, const uint16_t* x, const uint16_t* gamma, const uint16_t* beta, float eps,
                              const int8_t* Wq, long ldw, const float* sw, const float* bias, int N, int K, int n1,
                              uint16_t* out1, uint16_t* out2, int act2) {
  if (!x || !Wq || !sw || !out1 || (n1 < N && !out2)) return MX_ENULL;
  if ((gamma == nullptr) != (beta == nullptr)) return MX_ENULL;
  if (N < 1 || n1 < 0 || n1 > N || ldw < K || ldw % 16 || act2 < 0 || act2 > 2) return MX_ESHAPE;
  if (((uintptr_t)x | (uintptr_t)Wq) & 15) return MX_ELAYOUT;
  constexpr int R = 8;
  const dim3 g((N + 4 * R - 1) / (4 * R));
  if (K == 2048) hipLaunchKernelGGL((ln_gemv2_i8_kernel<2, R>), g, dim3(256), 0, st, x, gamma, beta, eps, Wq, ldw, sw, bias, N, n1, out1, out2, act2);
  else if (K == 1024) hipLaunchKernelGGL((ln_gemv2_i8_kernel<1, R>), g, dim3(256), 0, st, x, gamma, beta, eps, Wq, ldw, sw, bias, N, n1, out1, out2, act2);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// W8A8 fc2 (K2 = 8192 / 4096) and proj (Kp = 2048 / 1024) GEMVs + both residual adds: out = bf16(bf16(fc2(g)) +
// bf16(bf16(proj(a)) + xres)); W2 (N, K2) and Wp (N, Kp) int8, contiguous rows.
extern "C" int mx_gemv_dual_res_i8(hipStream_t st, const uint16_t* g, const int8_t* W2, const float* sw2,
                                   const float* b2, int K2, const uint16_t* a, const int8_t* Wp, const float* swp,
                                   const float* bp, int Kp, const uint16_t* xres, uint16_t* out, int N) {
  if (!g || !W2 || !sw2 || !b2 || !a || !Wp || !swp || !bp || !xres || !out) return MX_ENULL;
  if (N < 1) return MX_ESHAPE;
  if (((uintptr_t)g | (uintptr_t)W2 | (uintptr_t)a | (uintptr_t)Wp) & 15) return MX_ELAYOUT;
  constexpr int R = 2;
  const dim3 gr((N + 4 * R - 1) / (4 * R));
  if (K2 == 8192 && Kp == 2048)
    hipLaunchKernelGGL((gemv_dual_res_i8_kernel<8, 2, R>), gr, dim3(256), 0, st, g, W2, sw2, b2, a, Wp, swp, bp, xres, out, N);
  else if (K2 == 4096 && Kp == 1024)
    hipLaunchKernelGGL((gemv_dual_res_i8_kernel<4, 1, R>), gr, dim3(256), 0, st, g, W2, sw2, b2, a, Wp, swp, bp, xres, out, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// The W8A8 forms: W2 int8 (N, K2) with per-row scale sw2 (K2 = 8192 or 4096), Wp int8 (N, Kp) with swp (Kp = 2048 or
// 1024); g and a are quantised per token inside.
extern "C" int mx_decode_attn_fc2_i8(hipStream_t st, const uint16_t* qkv, const float* cs, uint16_t* kc, uint16_t* vc,
                                     int H, int ctx, const int* state, float scale, int S, float* part,
                                     uint16_t* attn_out, const uint16_t* g, const int8_t* W2, const float* sw2,
                                     const float* b2, int K2, uint16_t* y2, int N) {
  const int rc = attn_fc2_check(qkv, cs, kc, vc, state, H, ctx, S, part, attn_out, g, W2, b2, y2, N);
  if (rc != MX_OK) return rc;
  if (!sw2) return MX_ENULL;
  const dim3 gr(H * S + (N + DA_W - 1) / DA_W);
  const float sl2 = scale * 1.4426950408889634f;
  if (K2 == 8192)
    hipLaunchKernelGGL((attn_fc2_i8_kernel<8>), gr, dim3(64 * DA_W), 0, st, qkv, cs, kc, vc, H, ctx, state, sl2, S, part, attn_out, g, W2, sw2, b2, y2, N);
  else if (K2 == 4096)
    hipLaunchKernelGGL((attn_fc2_i8_kernel<4>), gr, dim3(64 * DA_W), 0, st, qkv, cs, kc, vc, H, ctx, state, sl2, S, part, attn_out, g, W2, sw2, b2, y2, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

extern "C" int mx_gemv_res2_i8(hipStream_t st, const uint16_t* y2, const uint16_t* a, int S, const float* part,
                               const int8_t* Wp, const float* swp, const float* bp, int Kp, const uint16_t* xres,
                               uint16_t* out, int N) {
  const int rc = res2_check(y2, a, S, part, Wp, bp, xres, out, N);
  if (rc != MX_OK) return rc;
  if (!swp) return MX_ENULL;
  constexpr int R = 2;
  const dim3 gr((N + 4 * R - 1) / (4 * R));
  if (Kp == 2048) hipLaunchKernelGGL((gemv_res2_i8_kernel<2, R>), gr, dim3(256), 0, st, y2, a, S, part, Wp, swp, bp, xres, out, N);
  else if (Kp == 1024) hipLaunchKernelGGL((gemv_res2_i8_kernel<1, R>), gr, dim3(256), 0, st, y2, a, S, part, Wp, swp, bp, xres, out, N);
  else return MX_ESHAPE;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
