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

// one workgroup per (batch row b, token t)
__global__ __launch_bounds__(256) void rope_kv_kernel(const uint16_t* __restrict__ qkv, long ldq,
                                                      const float* __restrict__ cs, uint16_t* __restrict__ q_out,
                                                      uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int n,
                                                      int H, int ctx, int pos0, int nslots, int bcast) {
  const int row = blockIdx.x;  // b * n + t
  const int b = row / n, t = row % n;
  const int pos = pos0 + t;
  const uint16_t* src = qkv + (long)row * ldq;
  const float* cp = cs + (long)pos * 32;  // (cos, sin) interleaved per frequency: [16][2]
  for (int i = threadIdx.x; i < H * 32; i += 256) {
    const int h = i >> 5, j = i & 31;
    // q and k: j < 16 -> rotated pair j ; j >= 16 -> pass-through dims 32 + 2 (j - 16), +1
    uint32_t qv, kv;
    int d;
    if (j < 16) {
      const float c = cp[2 * j], s = cp[2 * j + 1];
      float o0, o1;
      rot_pair(bf2f(src[h * 64 + j]), bf2f(src[h * 64 + 16 + j]), c, s, o0, o1);
      qv = pack2(o0, o1);
      rot_pair(bf2f(src[H * 64 + h * 64 + j]), bf2f(src[H * 64 + h * 64 + 16 + j]), c, s, o0, o1);
      kv = pack2(o0, o1);
      d = 2 * j;
    } else {
      d = 32 + 2 * (j - 16);
      qv = *reinterpret_cast<const uint32_t*>(src + h * 64 + d);
      kv = *reinterpret_cast<const uint32_t*>(src + H * 64 + h * 64 + d);
    }
    const uint32_t vv0 = *reinterpret_cast<const uint32_t*>(src + 2 * H * 64 + h * 64 + 2 * j);
    *reinterpret_cast<uint32_t*>(q_out + (((long)b * H + h) * n + t) * 64 + d) = qv;
    const int s0 = bcast ? 0 : b, s1 = bcast ? nslots : b + 1;
    for (int sl = s0; sl < s1; sl++) {
      const long base = (((long)sl * H + h) * ctx + pos) * 64;
      *reinterpret_cast<uint32_t*>(kc + base + d) = kv;
      *reinterpret_cast<uint32_t*>(vc + base + 2 * j) = vv0;
    }
  }
}

}  // namespace

// cs: (ctx_table, 16, 2) fp32 (cos, sin) table indexed by absolute position. Caches: [nslots][H][ctx][64].
// bcast = 1 writes the (B = 1) rows into every cache slot (image prefill shared by batched questions).
extern "C" int mx_rope_kv(hipStream_t st, const uint16_t* qkv, long ldq, const float* cs, uint16_t* q_out,
                          uint16_t* kc, uint16_t* vc, int B, int n, int H, int ctx, int pos0, int nslots, int bcast) {
  if (!qkv || !cs || !q_out || !kc || !vc) return MX_ENULL;
  if (B < 1 || n < 1 || H < 1 || pos0 < 0 || pos0 + n > ctx || ldq < 3L * H * 64 || ldq % 2) return MX_ESHAPE;
  if (bcast ? (B != 1 || nslots < 1) : (nslots < B)) return MX_ESHAPE;
  if (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)kc | (uintptr_t)vc) & 3) return MX_ELAYOUT;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(B * n), dim3(256), 0, st, qkv, ldq, cs, q_out, kc, vc, n, H, ctx, pos0,
                     nslots, bcast);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
