// Fused scaled-dot-product attention forward (QK^T -> online softmax -> PV) for head dims 64 and 72 on gfx950.
//
//   O[b, i, h, :] = sum_j softmax_j(scale * <Q[b,h,i,:], K[b,h,j,:]>) V[b,h,j,:]     over the visible keys j
//   key j is visible to query i (absolute position qpos0 + i) iff j < Tk and (j < causal_from or j <= qpos0 + i)
//   (causal_from >= Tk: no mask, the vision tower / TRecViT case; causal_from = prefix: the prompt prefill mask)
//
// Layout choices (MFMA 32x32x16, 64-wide waves):
//  * Each wave owns 32 queries. S^T = K Q^T is computed so that every lane holds the scores of ONE query
//    (column lane & 31) for 16 of every 32 keys; the other 16 sit in lane ^ 32. Row max / row sum therefore need a
//    single cross-half exchange, and the online-softmax rescale of the output is lane-local.
//  * O^T = V^T P^T: the score registers of S^T are, element for element, the B operand of this MFMA (the key
//    order inside a k-group is the same permutation on both operands), so P never goes through LDS.
//  * K is staged in LDS row-major [key][d] (row stride DK+8 bf16: conflict-free 16-byte operand reads); V is staged
//    transposed [d][key] (row stride 68 bf16: conflict-free 8-byte reads).
//  * Head dim 72 pads to 80 along the QK contraction (5 k-steps) and to 96 output rows for PV (3 row tiles).
// Numerics: fp32 scores and accumulators; P is rounded to bf16 before the PV product and the softmax denominator is
// summed over those rounded values, so numerator and denominator use the same weights.
#include "common.h"

namespace {

constexpr int KB = 64;        // keys per LDS block
constexpr int VS = KB + 4;    // V^T row stride (bf16)

template <int DK, int DV, int NW>
__global__ __launch_bounds__(64 * NW) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, long sq_b, long sq_h, long sq_t,
    const uint16_t* __restrict__ K, long sk_b, long sk_h, long sk_t,
    const uint16_t* __restrict__ V, long sv_b, long sv_h, long sv_t,
    uint16_t* __restrict__ O, long so_b, long so_h, long so_t,
    int Tq, int Tk, int D, float scale_log2, int qpos0, int causal_from) {
  constexpr int KS = DK + 8;
  constexpr int NT = 64 * NW;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[KB * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[DV * VS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, hk = lane >> 5;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qw0 = blockIdx.x * 32 * NW + wave * 32;
  const int qi = qw0 + lr;                       // this lane's query
  const int qpos = qpos0 + qi;
  const uint16_t* Qb = Q + b * sq_b + h * sq_h;
  const uint16_t* Kb = K + b * sk_b + h * sk_h;
  const uint16_t* Vb = V + b * sv_b + h * sv_h;

  // zero the padded rows of V^T once (they are never overwritten; their output rows are discarded)
  for (int i = tid; i < (DV - D) * VS; i += NT) Vt[D * VS + i] = 0;

  // Q operand in registers: k-step s covers d = 16 s + 8 hk .. +7
  bf16x8 qf[DK / 16];
  {
    const uint16_t* qrow = Qb + (long)min(qi, Tq - 1) * sq_t;
#pragma unroll
    for (int s = 0; s < DK / 16; s++) {
      const int d = 16 * s + 8 * hk;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (d < D) v = *reinterpret_cast<const u32x4*>(qrow + d);
      qf[s] = as_bf16x8(v);
    }
  }

  // keys this workgroup can see at all
  int kend = Tk;
  if (causal_from < Tk) {
    const int qlast = min(blockIdx.x * 32 * NW + 32 * NW, Tq) - 1;
    kend = min(Tk, max(causal_from, qpos0 + qlast + 1));
  }
  const int nkb = (kend + KB - 1) / KB;

  float m_run = -1e30f, l_run = 0.f;
  f32x16 oacc[DV / 32];
#pragma unroll
  for (int i = 0; i < DV / 32; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[i][e] = 0.f;

  const int dch = D / 8;  // 16-byte chunks per row
  for (int kb = 0; kb < nkb; kb++) {
    const int k0 = kb * KB;
    __syncthreads();
    // ---- stage K block [key][d], zero beyond Tk and beyond D (up to DK)
    for (int i = tid; i < KB * (DK / 8); i += NT) {
      const int key = i / (DK / 8), c = i % (DK / 8);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (k0 + key < Tk && c < dch) v = *reinterpret_cast<const u32x4*>(Kb + (long)(k0 + key) * sk_t + c * 8);
      *reinterpret_cast<u32x4*>(&Ks[key * KS + c * 8]) = v;
    }
    // ---- stage V block transposed [d][key]: each item = 4 keys x 8 d
    for (int i = tid; i < (KB / 4) * dch; i += NT) {
      const int g = i / dch, c = i % dch;
      u32x4 r[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int key = k0 + 4 * g + u;
        r[u] = (key < Tk) ? *reinterpret_cast<const u32x4*>(Vb + (long)key * sv_t + c * 8) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int w = e >> 1, sh = (e & 1) * 16;
        u32x2 o;
        o.x = ((r[0][w] >> sh) & 0xffffu) | (((r[1][w] >> sh) & 0xffffu) << 16);
        o.y = ((r[2][w] >> sh) & 0xffffu) | (((r[3][w] >> sh) & 0xffffu) << 16);
        *reinterpret_cast<u32x2*>(&Vt[(c * 8 + e) * VS + 4 * g]) = o;
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for 2 x 32 keys
    f32x16 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int e = 0; e < 16; e++) st[kt][e] = 0.f;
#pragma unroll
      for (int s = 0; s < DK / 16; s++) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(&Ks[(kt * 32 + lr) * KS + 16 * s + 8 * hk]));
        st[kt] = mfma32(a, qf[s], st[kt]);
      }
    }
    // ---- scale, mask, online softmax (lane = one query, 32 of the 64 keys; partner lane ^ 32 has the rest)
    const bool need_mask = (k0 + KB > Tk) || (causal_from < Tk && k0 + KB > causal_from && k0 + KB - 1 > qpos0 + qw0);
    float mx = -1e30f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        float v = st[kt][r] * scale_log2;
        if (need_mask) {
          const int key = k0 + kt * 32 + 8 * (r >> 2) + 4 * hk + (r & 3);
          if (!(key < Tk && (key < causal_from || key <= qpos))) v = -INFINITY;
        }
        st[kt][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - mnew);
    m_run = mnew;
    float sum = 0.f;
    uint32_t pk[2][8];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const uint16_t p0 = f2bf(exp2f(st[kt][r] - mnew)), p1 = f2bf(exp2f(st[kt][r + 1] - mnew));
        sum += bf2f(p0) + bf2f(p1);
        pk[kt][r >> 1] = (uint32_t)p0 | ((uint32_t)p1 << 16);
      }
    sum += __shfl_xor(sum, 32, 64);
    l_run = l_run * alpha + sum;
#pragma unroll
    for (int i = 0; i < DV / 32; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;

    // ---- O^T += V^T P^T ; k-step (kt, s) covers keys kt*32 + 16 s + {4hk..4hk+3, 8+4hk..8+4hk+3}
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        u32x4 pb = {pk[kt][4 * s], pk[kt][4 * s + 1], pk[kt][4 * s + 2], pk[kt][4 * s + 3]};
        const bf16x8 bp = as_bf16x8(pb);
        const int kk = kt * 32 + 16 * s + 4 * hk;
#pragma unroll
        for (int dt = 0; dt < DV / 32; dt++) {
          const uint16_t* vr = &Vt[(dt * 32 + lr) * VS + kk];
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vr);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 8);
          u32x4 va = {lo.x, lo.y, hi.x, hi.y};
          oacc[dt] = mfma32(as_bf16x8(va), bp, oacc[dt]);
        }
      }
  }

  if (qi >= Tq) return;
  const float inv = 1.f / l_run;
  uint16_t* orow = O + b * so_b + (long)qi * so_t + h * so_h;
#pragma unroll
  for (int dt = 0; dt < DV / 32; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = dt * 32 + 8 * g + 4 * hk;
      if (d < D) {
        u32x2 o;
        o.x = pack2(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv);
        o.y = pack2(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d) = o;
      }
    }
}

template <int DK, int DV, int NW>
hipError_t launch(hipStream_t st, const uint16_t* Q, long sq_b, long sq_h, long sq_t, const uint16_t* K, long sk_b,
                  long sk_h, long sk_t, const uint16_t* V, long sv_b, long sv_h, long sv_t, uint16_t* O, long so_b,
                  long so_h, long so_t, int B, int H, int Tq, int Tk, int D, float sl2, int qpos0, int causal_from) {
  dim3 g((Tq + 32 * NW - 1) / (32 * NW), H, B);
  hipLaunchKernelGGL((attn_fwd_kernel<DK, DV, NW>), g, dim3(64 * NW), 0, st, Q, sq_b, sq_h, sq_t, K, sk_b, sk_h, sk_t,
                     V, sv_b, sv_h, sv_t, O, so_b, so_h, so_t, Tq, Tk, D, sl2, qpos0, causal_from);
  return hipGetLastError();
}

}  // namespace

extern "C" int mx_sdpa_check(const void* Q, long sq_t, const void* K, long sk_t, const void* V, long sv_t,
                             const void* O, long so_t, int B, int H, int Tq, int Tk, int D) {
  if (!Q || !K || !V || !O) return MX_ENULL;
  if (D != 64 && D != 72) return MX_EBADCFG;
  if (B < 1 || H < 1 || Tq < 1 || Tk < 1) return MX_ESHAPE;
  if (sq_t % 8 || sk_t % 8 || sv_t % 8 || so_t % 4) return MX_ESHAPE;
  if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V) & 15) return MX_ELAYOUT;
  if ((uintptr_t)O & 7) return MX_ELAYOUT;
  return MX_OK;
}

// Strides are in elements; every batch/head stride must keep 16-byte alignment of the rows (multiples of 8).
extern "C" int mx_sdpa(hipStream_t st, const uint16_t* Q, long sq_b, long sq_h, long sq_t, const uint16_t* K,
                       long sk_b, long sk_h, long sk_t, const uint16_t* V, long sv_b, long sv_h, long sv_t, uint16_t* O,
                       long so_b, long so_h, long so_t, int B, int H, int Tq, int Tk, int D, float scale, int qpos0,
                       int causal_from) {
  int rc = mx_sdpa_check(Q, sq_t, K, sk_t, V, sv_t, O, so_t, B, H, Tq, Tk, D);
  if (rc) return rc;
  if ((sq_b | sq_h | sk_b | sk_h | sv_b | sv_h) % 8 || so_h % 4 || so_b % 4) return MX_ESHAPE;
  const float sl2 = scale * 1.4426950408889634f;
  // 4 waves (128 queries) per workgroup when that still gives >= 2 workgroups per CU, else 1 wave (32 queries)
  const long wg4 = (long)((Tq + 127) / 128) * H * B;
  hipError_t e;
  if (D == 72) {
    if (wg4 >= 512)
      e = launch<80, 96, 4>(st, Q, sq_b, sq_h, sq_t, K, sk_b, sk_h, sk_t, V, sv_b, sv_h, sv_t, O, so_b, so_h, so_t, B, H, Tq, Tk, D, sl2, qpos0, causal_from);
    else
      e = launch<80, 96, 1>(st, Q, sq_b, sq_h, sq_t, K, sk_b, sk_h, sk_t, V, sv_b, sv_h, sv_t, O, so_b, so_h, so_t, B, H, Tq, Tk, D, sl2, qpos0, causal_from);
  } else {
    if (wg4 >= 512)
      e = launch<64, 64, 4>(st, Q, sq_b, sq_h, sq_t, K, sk_b, sk_h, sk_t, V, sv_b, sv_h, sv_t, O, so_b, so_h, so_t, B, H, Tq, Tk, D, sl2, qpos0, causal_from);
    else
      e = launch<64, 64, 1>(st, Q, sq_b, sq_h, sq_t, K, sk_b, sk_h, sk_t, V, sv_b, sv_h, sv_t, O, so_b, so_h, so_t, B, H, Tq, Tk, D, sl2, qpos0, causal_from);
  }
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}
