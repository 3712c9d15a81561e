// Partial rotary embedding + KV-cache write for the moondream2 text model (head_dim 64, rotary dim 32).
//
// Rotation (moondream's apply_rotary_emb, restated in md2fast._rope and fused.py:53-58): for each head, with
// a = x[0:16], b = x[16:32] (non-interleaved halves) and (c, s) = freqs_cis[pos, 0:16]:
//     out[2j]   = a_j c_j - b_j s_j        out[2j+1] = a_j s_j + b_j c_j          (j < 16, interleaved output)
//     out[32:64] = x[32:64]
// computed in fp32 (bf16 inputs promoted, two products rounded to fp32 then subtracted/added) and rounded to bf16.
//
// Prefill form: rows t of a fused qkv matrix (q | k | v, each H x 64) at positions pos0 + t.
//   q -> q_out [B][H][n][64] (contiguous), rotated k and raw v -> caches [slot][H][ctx][64] at position pos0 + t.
#include "common.h"

namespace {

__device__ __forceinline__ void rot_pair(float a, float b, float c, float s, float& o0, float& o1) {
  o0 = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
  o1 = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
}

// One workgroup per (batch row b, token t); thread (head h, unit u < 4) moves 16-byte chunks 2u and 2u + 1 of the
// head's q, k and v (dims 16u .. 16u + 15 of the output): units 0 and 1 rotate the pairs j = 8u .. 8u + 7
// (a = x[j] from input chunk u, b = x[16 + j] from chunk u + 2), units 2 and 3 pass dims 32 .. 63 through. Every load
// of a thread is issued before its arithmetic, so a row is one memory round trip.
__global__ __launch_bounds__(128) void rope_kv_kernel(const uint16_t* __restrict__ qkv, long ldq,
                                                      const float* __restrict__ cs, uint16_t* __restrict__ q_out,
                                                      uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int n,
                                                      int H, int ctx, int pos0, int nslots, int bcast) {
  const int row = blockIdx.x;  // b * n + t
  const int b = row / n, t = row % n;
  const int pos = pos0 + t;
  const uint16_t* src = qkv + (long)row * ldq;
  const float* cp = cs + (long)pos * 32;  // (cos, sin) interleaved per frequency: [16][2]
  const int s0 = bcast ? 0 : b, s1 = bcast ? nslots : b + 1;
  for (int i = threadIdx.x; i < H * 4; i += 128) {
    const int h = i >> 2, u = i & 3;
    const uint16_t* qh = src + h * 64;
    const uint16_t* kh = src + (H + h) * 64;
    const uint16_t* vh = src + (2 * H + h) * 64;
    const bool rot = u < 2;
    // rotated units read input chunks u and u + 2, pass-through units their own chunks 2u and 2u + 1
    const int c0 = rot ? u : 2 * u, c1 = rot ? u + 2 : 2 * u + 1;
    const u32x4 qa = *reinterpret_cast<const u32x4*>(qh + 8 * c0), qb = *reinterpret_cast<const u32x4*>(qh + 8 * c1);
    const u32x4 ka = *reinterpret_cast<const u32x4*>(kh + 8 * c0), kb = *reinterpret_cast<const u32x4*>(kh + 8 * c1);
    const u32x4 v0 = *reinterpret_cast<const u32x4*>(vh + 16 * u), v1 = *reinterpret_cast<const u32x4*>(vh + 16 * u + 8);
    f32x4 cv[4];
#pragma unroll
    for (int m = 0; m < 4; m++) cv[m] = *reinterpret_cast<const f32x4*>(cp + 16 * (u & 1) + 4 * m);
    u32x4 q0 = qa, q1 = qb, k0 = ka, k1 = kb;
    if (rot) {
      uint32_t qo[8], ko[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float c = cv[e >> 1][2 * (e & 1)], sn = cv[e >> 1][2 * (e & 1) + 1];  // cp[2j], cp[2j + 1], j = 8u + e
        const uint32_t wa = qa[e >> 1], wb = qb[e >> 1], xa = ka[e >> 1], xb = kb[e >> 1];
        const float a = (e & 1) ? hi_bf(wa) : lo_bf(wa), bq = (e & 1) ? hi_bf(wb) : lo_bf(wb);
        const float ak = (e & 1) ? hi_bf(xa) : lo_bf(xa), bk = (e & 1) ? hi_bf(xb) : lo_bf(xb);
        float o0, o1;
        rot_pair(a, bq, c, sn, o0, o1);
        qo[e] = pack2(o0, o1);
        rot_pair(ak, bk, c, sn, o0, o1);
        ko[e] = pack2(o0, o1);
      }
      q0 = u32x4{qo[0], qo[1], qo[2], qo[3]};
      q1 = u32x4{qo[4], qo[5], qo[6], qo[7]};
      k0 = u32x4{ko[0], ko[1], ko[2], ko[3]};
      k1 = u32x4{ko[4], ko[5], ko[6], ko[7]};
    }
    uint16_t* qd = q_out + (((long)b * H + h) * n + t) * 64 + 16 * u;
    *reinterpret_cast<u32x4*>(qd) = q0;
    *reinterpret_cast<u32x4*>(qd + 8) = q1;
    for (int sl = s0; sl < s1; sl++) {
      const long base = (((long)sl * H + h) * ctx + pos) * 64 + 16 * u;
      *reinterpret_cast<u32x4*>(kc + base) = k0;
      *reinterpret_cast<u32x4*>(kc + base + 8) = k1;
      *reinterpret_cast<u32x4*>(vc + base) = v0;
      *reinterpret_cast<u32x4*>(vc + base + 8) = v1;
    }
  }
}

}  // namespace

// cs: (ctx_table, 16, 2) fp32 (cos, sin) table indexed by absolute position. Caches: [nslots][H][ctx][64]. qkv rows
// (ldq a multiple of 8), cs, q_out and the caches 16-byte aligned.
// bcast = 1 writes the (B = 1) rows into every cache slot (image prefill shared by batched questions).
extern "C" int mx_rope_kv(hipStream_t st, const uint16_t* qkv, long ldq, const float* cs, uint16_t* q_out,
                          uint16_t* kc, uint16_t* vc, int B, int n, int H, int ctx, int pos0, int nslots, int bcast) {
  if (!qkv || !cs || !q_out || !kc || !vc) return MX_ENULL;
  if (B < 1 || n < 1 || H < 1 || pos0 < 0 || pos0 + n > ctx || ldq < 3L * H * 64 || ldq % 2) return MX_ESHAPE;
  if (bcast ? (B != 1 || nslots < 1) : (nslots < B)) return MX_ESHAPE;
  if (((uintptr_t)qkv | (uintptr_t)cs | (uintptr_t)q_out | (uintptr_t)kc | (uintptr_t)vc) & 15 || ldq % 8)
    return MX_ELAYOUT;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(B * n), dim3(128), 0, st, qkv, ldq, cs, q_out, kc, vc, n, H, ctx, pos0,
                     nslots, bcast);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
