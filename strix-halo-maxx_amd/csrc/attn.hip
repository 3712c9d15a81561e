// Fused scaled-dot-product attention forward (QK^T -> online softmax -> PV) for head dims 64 and 72 on gfx950.
//
//   O[b, i, h, :] = sum_j softmax_j(scale * <Q[b,h,i,:], K[b,h,j,:]>) V[b,h,j,:]     over the visible keys j
//   key j is visible to query i (absolute position qpos0 + i) iff j < Tk and (j < causal_from or j <= qpos0 + i)
//   (causal_from >= Tk: no mask, the vision tower / TRecViT case; causal_from = prefix: the prompt prefill mask)
//
// Layout choices (MFMA 32x32x16, 64-wide waves):
//  * A query wave owns 32 queries. S^T = K Q^T is computed so that every lane holds the scores of ONE query
//    (column lane & 31) for 16 of every 32 keys; the other 16 sit in lane ^ 32. Row max / row sum need a single
//    cross-half exchange, and the online-softmax rescale of the output is lane-local.
//  * O^T = V^T P^T: the score registers of S^T are, element for element, the B operand of this MFMA (the key
//    order inside a k-group is the same permutation on both operands), so P never goes through LDS.
//  * K is staged in LDS row-major [key][d] (row stride DK+8 bf16: conflict-free 16-byte operand reads); V is staged
//    transposed [d][key] (row stride KB+4: conflict-free 8-byte reads). The next key block is prefetched into
//    registers while the current one is consumed.
//  * Workgroup = NQW query waves x NKW key waves. With NKW > 1 the key blocks are dealt round-robin to the key
//    waves (each with its own LDS staging) and the partial (max, sum, O) of each query are merged at the end in fp32:
//    this is how batch-1 shapes (16 heads x 729 queries = 368 query waves) still put >1000 waves on 256 CUs.
//  * Head dim 72 pads to 80 along the QK contraction (5 k-steps) and to 96 output rows for PV (3 row tiles).
// Numerics: fp32 scores and accumulators; P is rounded to bf16 before the PV product and the softmax denominator is
// summed over those rounded values, so numerator and denominator use the same weights.
#include "common.h"

namespace {

template <int DK, int DV, int NQW, int NKW, int KB>
struct AttnSmem {
  static constexpr int KS = DK + 8, VS = KB + 4;
  static constexpr int GROUP = KB * KS + DV * VS;              // bf16 elements per key group
  static constexpr int STAGE_BYTES = NKW * GROUP * 2;
  static constexpr int COMB_BYTES = NKW > 1 ? NKW * NQW * (2 * 32 + (DV / 32) * 16 * 64) * 4 : 0;
  static constexpr int BYTES = STAGE_BYTES > COMB_BYTES ? STAGE_BYTES : COMB_BYTES;
};

template <int DK, int DV, int NQW, int NKW, int KB>
__global__ __launch_bounds__(64 * NQW * NKW) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, long sq_b, long sq_h, long sq_t,
    const uint16_t* __restrict__ K, long sk_b, long sk_h, long sk_t,
    const uint16_t* __restrict__ V, long sv_b, long sv_h, long sv_t,
    uint16_t* __restrict__ O, long so_b, long so_h, long so_t,
    int Tq, int Tk, int D, float scale_log2, int qpos0, int causal_from) {
  using SM = AttnSmem<DK, DV, NQW, NKW, KB>;
  constexpr int KS = SM::KS, VS = SM::VS;
  constexpr int GT = 64 * NQW;                    // threads per key group (they stage that group's blocks)
  constexpr int KCH = DK / 8;                     // 16-byte chunks per staged K row
  constexpr int KI = (KB * KCH + GT - 1) / GT;    // K chunks per thread
  constexpr int VG = KB / 4;                      // 4-key groups per block
  constexpr int VI = (VG * 9 + GT - 1) / GT;      // V items (4 keys x 8 d) per thread, d <= 72
  constexpr int NST = KB / 32;                    // S^T tiles per block
  __shared__ __attribute__((aligned(16))) uint16_t smem[SM::BYTES / 2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qg = wave % NQW, kw = wave / NQW;
  const int gtid = qg * 64 + lane;
  const int lr = lane & 31, hk = lane >> 5;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qw0 = blockIdx.x * 32 * NQW + qg * 32;
  const int qi = qw0 + lr;
  const int qpos = qpos0 + qi;
  const uint16_t* Qb = Q + b * sq_b + h * sq_h;
  const uint16_t* Kb = K + b * sk_b + h * sk_h;
  const uint16_t* Vb = V + b * sv_b + h * sv_h;
  uint16_t* Ks = smem + kw * SM::GROUP;
  uint16_t* Vt = Ks + KB * KS;
  const int dch = D >> 3;

  for (int i = gtid; i < (DV - D) * VS; i += GT) Vt[D * VS + i] = 0;

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

  int kend = Tk;
  if (causal_from < Tk) {
    const int qlast = min((int)(blockIdx.x + 1) * 32 * NQW, Tq) - 1;
    kend = min(Tk, max(causal_from, qpos0 + qlast + 1));
  }
  const int nkb = (kend + KB - 1) / KB;
  const int nrounds = (nkb + NKW - 1) / NKW;

  // ---- staging registers for one key block of this key group
  u32x4 kr[KI];
  u32x4 vr[VI][4];
  auto load_block = [&](int kb) {
    const int k0 = kb * KB;
#pragma unroll
    for (int j = 0; j < KI; j++) {
      const int i = gtid + j * GT;
      const int key = i / KCH, c = i % KCH;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (i < KB * KCH && k0 + key < Tk && c < dch) v = *reinterpret_cast<const u32x4*>(Kb + (long)(k0 + key) * sk_t + c * 8);
      kr[j] = v;
    }
#pragma unroll
    for (int j = 0; j < VI; j++) {
      const int i = gtid + j * GT;
      const int g = i / 9, c = i % 9;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int key = k0 + 4 * g + u;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (i < VG * 9 && c < dch && key < Tk) v = *reinterpret_cast<const u32x4*>(Vb + (long)key * sv_t + c * 8);
        vr[j][u] = v;
      }
    }
  };
  auto store_block = [&]() {
#pragma unroll
    for (int j = 0; j < KI; j++) {
      const int i = gtid + j * GT;
      if (i < KB * KCH) *reinterpret_cast<u32x4*>(&Ks[(i / KCH) * KS + (i % KCH) * 8]) = kr[j];
    }
#pragma unroll
    for (int j = 0; j < VI; j++) {
      const int i = gtid + j * GT;
      const int g = i / 9, c = i % 9;
      if (i < VG * 9 && c < dch) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int w = e >> 1, sh = (e & 1) * 16;
          u32x2 o;
          o.x = ((vr[j][0][w] >> sh) & 0xffffu) | (((vr[j][1][w] >> sh) & 0xffffu) << 16);
          o.y = ((vr[j][2][w] >> sh) & 0xffffu) | (((vr[j][3][w] >> sh) & 0xffffu) << 16);
          *reinterpret_cast<u32x2*>(&Vt[(c * 8 + e) * VS + 4 * g]) = o;
        }
      }
    }
  };

  float m_run = -1e30f, l_run = 0.f;
  f32x16 oacc[DV / 32];
#pragma unroll
  for (int i = 0; i < DV / 32; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[i][e] = 0.f;

  if (kw < nkb) load_block(kw);
  for (int r = 0; r < nrounds; r++) {
    const int kb = r * NKW + kw;
    __syncthreads();
    if (kb < nkb) store_block();
    __syncthreads();
    if (kb + NKW < nkb) load_block(kb + NKW);
    if (kb >= nkb) continue;
    const int k0 = kb * KB;

    // ---- S^T = K Q^T for NST x 32 keys
    f32x16 st[NST];
#pragma unroll
    for (int kt = 0; kt < NST; kt++) {
#pragma unroll
      for (int e = 0; e < 16; e++) st[kt][e] = 0.f;
#pragma unroll
      for (int s = 0; s < DK / 16; s++) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(&Ks[(kt * 32 + lr) * KS + 16 * s + 8 * hk]));
        st[kt] = mfma32(a, qf[s], st[kt]);
      }
    }
    // ---- scale, mask, online softmax
    const bool need_mask = (k0 + KB > Tk) || (causal_from < Tk && k0 + KB > causal_from && k0 + KB - 1 > qpos0 + qw0);
    float mx = -1e30f;
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int r2 = 0; r2 < 16; r2++) {
        float v = st[kt][r2] * scale_log2;
        if (need_mask) {
          const int key = k0 + kt * 32 + 8 * (r2 >> 2) + 4 * hk + (r2 & 3);
          if (!(key < Tk && (key < causal_from || key <= qpos))) v = -INFINITY;
        }
        st[kt][r2] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
    m_run = mnew;
    float sum = 0.f;
    uint32_t pk[NST][8];
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int r2 = 0; r2 < 16; r2 += 2) {
        const uint32_t w = pack2(__builtin_amdgcn_exp2f(st[kt][r2] - mnew), __builtin_amdgcn_exp2f(st[kt][r2 + 1] - mnew));
        sum += lo_bf(w) + hi_bf(w);
        pk[kt][r2 >> 1] = w;
      }
    sum += __shfl_xor(sum, 32, 64);
    l_run = l_run * alpha + sum;
#pragma unroll
    for (int i = 0; i < DV / 32; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;

    // ---- O^T += V^T P^T ; k-step (kt, s) covers keys kt*32 + 16 s + {4hk..4hk+3, 8+4hk..8+4hk+3}
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        u32x4 pb = {pk[kt][4 * s], pk[kt][4 * s + 1], pk[kt][4 * s + 2], pk[kt][4 * s + 3]};
        const bf16x8 bp = as_bf16x8(pb);
        const int kk = kt * 32 + 16 * s + 4 * hk;
#pragma unroll
        for (int dt = 0; dt < DV / 32; dt++) {
          const uint16_t* vrow = &Vt[(dt * 32 + lr) * VS + kk];
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
          u32x4 va = {lo.x, lo.y, hi.x, hi.y};
          oacc[dt] = mfma32(as_bf16x8(va), bp, oacc[dt]);
        }
      }
  }

  if constexpr (NKW > 1) {
    // ---- merge the key waves' partial results (fp32) through LDS
    constexpr int OW = (DV / 32) * 16 * 64;  // floats of O per wave
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + NKW * NQW * 32;
    float* co = cl + NKW * NQW * 32;
    __syncthreads();
    const int slot = kw * NQW + qg;
    if (hk == 0) { cm[slot * 32 + lr] = m_run; cl[slot * 32 + lr] = l_run; }
#pragma unroll
    for (int dt = 0; dt < DV / 32; dt++)
#pragma unroll
      for (int e = 0; e < 16; e++) co[slot * OW + (dt * 16 + e) * 64 + lane] = oacc[dt][e];
    __syncthreads();
    if (kw != 0) return;
    float M = -1e30f;
#pragma unroll
    for (int k = 0; k < NKW; k++) M = fmaxf(M, cm[(k * NQW + qg) * 32 + lr]);
    float L = 0.f;
#pragma unroll
    for (int dt = 0; dt < DV / 32; dt++)
#pragma unroll
      for (int e = 0; e < 16; e++) oacc[dt][e] = 0.f;
#pragma unroll
    for (int k = 0; k < NKW; k++) {
      const int sl = k * NQW + qg;
      const float f = __builtin_amdgcn_exp2f(cm[sl * 32 + lr] - M);
      L += cl[sl * 32 + lr] * f;
#pragma unroll
      for (int dt = 0; dt < DV / 32; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[dt][e] += co[sl * OW + (dt * 16 + e) * 64 + lane] * f;
    }
    l_run = L;
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

struct Args {
  const uint16_t *Q, *K, *V;
  uint16_t* O;
  long sq_b, sq_h, sq_t, sk_b, sk_h, sk_t, sv_b, sv_h, sv_t, so_b, so_h, so_t;
  int B, H, Tq, Tk, D, qpos0, causal_from;
  float sl2;
};

template <int DK, int DV, int NQW, int NKW, int KB>
hipError_t launch(hipStream_t st, const Args& a) {
  dim3 g((a.Tq + 32 * NQW - 1) / (32 * NQW), a.H, a.B);
  hipLaunchKernelGGL((attn_fwd_kernel<DK, DV, NQW, NKW, KB>), g, dim3(64 * NQW * NKW), 0, st, a.Q, a.sq_b, a.sq_h,
                     a.sq_t, a.K, a.sk_b, a.sk_h, a.sk_t, a.V, a.sv_b, a.sv_h, a.sv_t, a.O, a.so_b, a.so_h, a.so_t,
                     a.Tq, a.Tk, a.D, a.sl2, a.qpos0, a.causal_from);
  return hipGetLastError();
}

}  // namespace

extern "C" int mx_sdpa_check(const void* Q, long sq_t, const void* K, long sk_t, const void* V, long sv_t,
                             const void* O, long so_t, int B, int H, int Tq, int Tk, int D) {
  if (!Q || !K || !V || !O) return MX_ENULL;
  if (D != 64 && D != 72) return MX_EBADCFG;
  if (B < 1 || H < 1 || Tq < 1 || Tk < 1 || H > 65535 || B > 65535) return MX_ESHAPE;
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
  const Args a{Q, K, V, O, sq_b, sq_h, sq_t, sk_b, sk_h, sk_t, sv_b, sv_h, sv_t, so_b, so_h, so_t,
               B, H, Tq, Tk, D, qpos0, causal_from, scale * 1.4426950408889634f};
  // many (batch, head, 128-query) tiles: 4 query waves share each staged key block; few: split the keys over
  // 4 waves per 32 queries so the grid still fills the GPU
  const long wg4 = (long)((Tq + 127) / 128) * H * B;
  hipError_t e;
  if (D == 72) e = (wg4 >= 512) ? launch<80, 96, 4, 1, 64>(st, a) : launch<80, 96, 1, 4, 32>(st, a);
  else e = (wg4 >= 512) ? launch<64, 64, 4, 1, 64>(st, a) : launch<64, 64, 1, 4, 32>(st, a);
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}
