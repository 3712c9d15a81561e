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
//  * K and V blocks of KB keys are copied row-major ([key][d], 2 D bytes per row) into an S-stage LDS ring by the
//    asynchronous LDS-DMA load, one or more blocks ahead of the MFMAs; every wave of the workgroup issues a share of
//    each block's 16-byte chunks. The V^T operand of the PV product is read straight from the row-major block with
//    the LDS transpose read (ds_read_b64_tr_b16). D = 64 rows are 128 bytes: their 16-byte chunks are XOR-swizzled
//    by ((key >> 1) & 7) (the DMA fetches the global chunk that belongs at each slot) so operand reads spread over
//    the 64 banks; D = 72 rows (144 bytes) need no swizzle.
//  * Workgroup = NQW query waves x NKW key waves. Each KB-key block is split into NKW sub-blocks of KB / NKW keys;
//    key wave w consumes sub-block w of every block, and the partial (max, sum, O) of each query are merged at the
//    end in fp32. Workgroups of 4, 8 or 16 waves; small grids (batch-1 shapes: 16 heads x 729 queries) use NKW = 4.
//  * Head dim 72 pads to 80 along the QK contraction (5 k-steps; Q's padding is zero, so the neighbouring LDS bytes
//    that K's padding reads are multiplied by 0) and to 96 output rows for PV (3 row tiles; rows >= 72 are dropped).
// Numerics: fp32 scores and accumulators; P is rounded to bf16 before the PV product and the softmax denominator is
// summed over those rounded values, so numerator and denominator use the same weights. With D = 72 the PV product
// computes the denominator itself: the V^T operand rows 72..95 (padding, dropped) are replaced by ones, so those
// output rows accumulate sum_j P[i, j] in fp32 inside the MFMA (and are rescaled with O), which takes the per-score
// unpack-and-add off the VALU, the unit that bounds the small-grid shapes.
#include "common.h"

namespace {

template <int D, int NQW, int NKW, int KB, int S>
struct AttnCfg {
  static constexpr int DK = D == 72 ? 80 : 64;      // QK contraction (multiple of 16)
  static constexpr int DV = D == 72 ? 96 : 64;      // PV output rows (multiple of 32)
  static constexpr int CPR = D / 8;                 // 16-byte chunks per K / V row
  static constexpr bool SWZ = (D == 64);
  static constexpr int KBW = KB / NKW;              // keys per key wave per block
  static constexpr int NST = KBW / 32;              // S^T tiles per key wave per block
  static constexpr int NW = NQW * NKW;              // waves per workgroup
  static constexpr int NCH = 2 * KB * CPR;          // K + V chunks per block
  static constexpr int NI = (NCH + 63) / 64;        // DMA instructions per block
  static constexpr int NIW = (NI + NW - 1) / NW;    // ... per wave (instructions >= NI are padding)
  // one ring stage: K block, V block (NI KB together), then a 1 KB landing slot that every padding instruction
  // writes (the same bytes: the block's first chunk), which also absorbs the last rows' over-reads (PV rows 72..95
  // of D = 72; the QK over-read of K's last row, chunk 9 of D = 72, lands in the V block)
  static constexpr int STAGE_B = NI * 1024 + 1024;
  static constexpr int RING_B = S * STAGE_B;
  // O registers per lane that hold output rows < D (register u: tile u / 16, row 32 (u / 16) + 8 ((u % 16) / 4) +
  // 4 (lane >> 5) + u % 4): all 32 for D = 64, tiles 0-1 and the first 4 registers of tile 2 for D = 72
  static constexpr int NU = D == 72 ? 36 : 32;
  static constexpr int COMB_B = NKW > 1 ? NW * (2 + NU) * 64 * 4 : 0;
  static constexpr int BYTES = RING_B > COMB_B ? RING_B : COMB_B;
  static_assert(KBW % 32 == 0 && NST >= 1, "key sub-block of whole 32-key tiles");
  static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves");
  static_assert(BYTES <= 160 * 1024, "LDS");
  static_assert(D == 64 || D == 72, "head dim");
};

template <int D, int NQW, int NKW, int KB, int S>
__global__ __launch_bounds__(64 * NQW * NKW) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, long sq_b, long sq_h, long sq_t,
    const uint16_t* __restrict__ K, long sk_b, long sk_h, long sk_t,
    const uint16_t* __restrict__ V, long sv_b, long sv_h, long sv_t,
    uint16_t* __restrict__ O, long so_b, long so_h, long so_t,
    int Tq, int Tk, int H, int nbh, float scale_log2, int qpos0, int causal_from) {
  using C = AttnCfg<D, NQW, NKW, KB, S>;
  constexpr int DK = C::DK, DV = C::DV, CPR = C::CPR, KBW = C::KBW, NST = C::NST, NIW = C::NIW;
  constexpr int ROWB = 2 * D;  // bytes per staged row
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave % NQW, kw = wave / NQW;
  const int lr = lane & 31, hk = lane >> 5;
  // Tiles (query tile x, head h, batch b) in a 1-D grid. The dispatcher sends workgroup i to XCD i % 8; consecutive
  // tile numbers (the query tiles of one head first) are placed on one XCD so each head's K / V is fetched into a
  // single XCD's L2.
  const int nqt = (Tq + 32 * NQW - 1) / (32 * NQW);
  const int ntile = nqt * nbh;
  const int per = ntile / 8, rem = ntile % 8, xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
  const int tnum = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int qx = tnum % nqt, bh = tnum / nqt;
  const int b = bh / H, h = bh % H;
  const int qw0 = qx * 32 * NQW + qg * 32;
  const int qi = qw0 + lr;
  const int qpos = qpos0 + qi;
  const uint16_t* Qb = Q + b * sq_b + h * sq_h;
  const uint16_t* Kb = K + b * sk_b + h * sk_h;
  const uint16_t* Vb = V + b * sv_b + h * sv_h;
  const uint32_t sbase = lds_off(smem);

  int kend = Tk;
  if (causal_from < Tk) {
    const int qlast = min((qx + 1) * 32 * NQW, Tq) - 1;
    kend = min(Tk, max(causal_from, qpos0 + qlast + 1));
  }
  const int nkb = (kend + KB - 1) / KB;

  // ---- this lane's DMA chunks: instruction q = wave + NW i of a block covers chunks 64 q .. 64 q + 63, which are all
  // K chunks (q < KB * CPR / 64) or all V chunks; instructions q >= NI are padding and refetch the block's first chunk
  // into the stage's landing slot
  static_assert((KB * CPR) % 64 == 0, "an instruction never straddles the K and V parts");
  constexpr int NIK = KB * CPR / 64;  // K instructions per block
  uint32_t doff[NIW];                 // byte offset of this lane's chunk from the block's first row
  int dkey[NIW];                      // its key within the block
#pragma unroll
  for (int i = 0; i < NIW; i++) {
    const int q = wave + C::NW * i;
    const int ch = q < C::NI ? (q * 64 + lane) % (KB * CPR) : 0;
    const int key = ch / CPR, slot = ch % CPR;
    const int c = C::SWZ ? (slot ^ ((key >> 1) & 7)) : slot;
    const long st_el = (q >= NIK && q < C::NI) ? sv_t : sk_t;
    dkey[i] = key;
    doff[i] = (uint32_t)(key * st_el * 2 + c * 16);
  }
  // rows past the last key are clamped to it (finite data; those keys are masked)
  auto issue = [&](int kb, int st) {
    const uint32_t base = sbase + (uint32_t)(st * C::STAGE_B);
    const uint16_t* kbase = Kb + (long)kb * KB * sk_t;
    const uint16_t* vbase = Vb + (long)kb * KB * sv_t;
    const int lim = Tk - 1 - kb * KB;  // last valid key within the block
    if (lim >= KB - 1) {
#pragma unroll
      for (int i = 0; i < NIW; i++) {
        const int q = wave + C::NW * i;
        dma16s((q >= NIK && q < C::NI) ? vbase : kbase, doff[i], base + min(q, C::NI) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NIW; i++) {
        const int q = wave + C::NW * i;
        const bool isv = q >= NIK && q < C::NI;
        const long st_el = isv ? sv_t : sk_t;
        const int key = dkey[i];
        const uint32_t off = doff[i] - (uint32_t)((key > lim ? key - lim : 0) * st_el * 2);
        dma16s(isv ? vbase : kbase, off, base + min(q, C::NI) * 1024);
      }
    }
  };

  // D = 72: the PV operand's padding rows carry ones, and O^T row 72 (+ 4 hk) = register 4 of the last row tile holds
  // the denominator; D = 64 has no padding rows and sums the rounded P on the VALU
  constexpr bool ONES = DV > D;
  static_assert(!ONES || DV - 32 + 8 >= D, "register 4 of the last row tile is a padding row");
  const bool ones_lane = ONES && (lane & 31) >= D - (DV - 32);
  float m_run = -1e30f, l_run = 0.f;
  bool first = true;  // no key block consumed yet by this wave (O and l are still zero)
  f32x16 oacc[DV / 32];
#pragma unroll
  for (int i = 0; i < DV / 32; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[i][e] = 0.f;

  // Stage 0, then this lane's Q fragments, then one wait for both, then the other prefetched stages. The compiler
  // does not count the LDS-DMA loads (inline asm), so a Q fragment still in flight at its first use would make it wait
  // with a count that assumes nothing was issued after Q, i.e. for every prefetched stage, on every pass of the key
  // loop; waiting for Q here (a wait the compiler sees) leaves the loop with the ring's own waits only.
  if (nkb > 0) issue(0, 0);
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
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0); expcnt, lgkmcnt not waited (gfx9 encoding)
#pragma unroll
  for (int s = 1; s < S - 1; s++)
    if (s < nkb) issue(s, s);

  for (int kb = 0; kb < nkb; kb++) {
    wait_stages<NIW, S - 2>(nkb - 1 - kb);
    __syncthreads();
    if (kb + S - 1 < nkb) issue(kb + S - 1, (kb + S - 1) % S);
    const int k0 = kb * KB + kw * KBW;  // first key of this wave's sub-block
    if (k0 >= kend) continue;
    const uint8_t* Kst = smem + (kb % S) * C::STAGE_B + kw * KBW * ROWB;
    const uint8_t* Vst = smem + (kb % S) * C::STAGE_B + KB * ROWB + kw * KBW * ROWB;

    // ---- S^T = K Q^T for NST x 32 keys (the NST chains interleave)
    f32x16 st[NST];
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int e = 0; e < 16; e++) st[kt][e] = 0.f;
#pragma unroll
    for (int s = 0; s < DK / 16; s++)
#pragma unroll
      for (int kt = 0; kt < NST; kt++) {
        const int key = kt * 32 + lr;  // within the sub-block; the swizzle uses the key within the block
        const int c = 2 * s + hk;
        const int slot = C::SWZ ? (c ^ (((kw * KBW + key) >> 1) & 7)) : c;
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(Kst + key * ROWB + slot * 16));
        st[kt] = mfma32(a, qf[s], st[kt]);
      }
    // ---- mask, online softmax. Scores stay unscaled until the exponent: p = exp2(scale_log2 s - m) with m the
    // running max in scaled units. The running max is only raised (and O, l rescaled) when a query's block max
    // exceeds it by more than 8, i.e. the exponentials of a stale max stay <= 256; the normalisation at the end is
    // unaffected.
    const bool need_mask = (k0 + KBW > Tk) || (causal_from < Tk && k0 + KBW > causal_from && k0 + KBW - 1 > qpos0 + qw0);
    float mx = -INFINITY;
    if (need_mask) {
      const int lim = min(Tk, max(causal_from, qpos + 1));  // keys < lim are visible to this query
#pragma unroll
      for (int kt = 0; kt < NST; kt++)
#pragma unroll
        for (int r2 = 0; r2 < 16; r2++) {
          const int key = k0 + kt * 32 + 8 * (r2 >> 2) + 4 * hk + (r2 & 3);
          const float v = key < lim ? st[kt][r2] : -INFINITY;
          st[kt][r2] = v;
          mx = fmaxf(mx, v);
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < NST; kt++)
#pragma unroll
        for (int r2 = 0; r2 < 16; r2++) mx = fmaxf(mx, st[kt][r2]);
    }
    mx = halves_max(mx) * scale_log2;
    const bool grow = mx > m_run + 8.f;
    if (__any(grow)) {
      const float mnew = grow ? mx : m_run;
      if (!first) {
        const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
        if constexpr (!ONES) l_run *= alpha;
#pragma unroll
        for (int i = 0; i < DV / 32; i++)
#pragma unroll
          for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;
      }
      m_run = mnew;
    }
    first = false;
    float sum = 0.f;
    uint32_t pk[NST][8];
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int r2 = 0; r2 < 16; r2 += 2) {
        const uint32_t w = pack2(__builtin_amdgcn_exp2f(__builtin_fmaf(st[kt][r2], scale_log2, -m_run)),
                                 __builtin_amdgcn_exp2f(__builtin_fmaf(st[kt][r2 + 1], scale_log2, -m_run)));
        if constexpr (!ONES) sum += lo_bf(w) + hi_bf(w);
        pk[kt][r2 >> 1] = w;
      }
    if constexpr (!ONES) l_run += halves_sum(sum);

    // ---- O^T += V^T P^T ; k-step (kt, s) covers keys kt*32 + 16 s + {4hk..4hk+3, 8+4hk..8+4hk+3}. The V^T
    // operand comes from two transpose reads: lane j = lane & 15 of each 16-lane group points at
    // V[first key + (j >> 2)][d0 + 4 (j & 3)], d0 = 32 dt + 16 ((lane >> 4) & 1).
    const int jr = (lane & 15) >> 2, jc = 4 * (lane & 3) + 16 * ((lane >> 4) & 1);
#pragma unroll
    for (int kt = 0; kt < NST; kt++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const u32x4 pb = {pk[kt][4 * s], pk[kt][4 * s + 1], pk[kt][4 * s + 2], pk[kt][4 * s + 3]};
        const bf16x8 bp = as_bf16x8(pb);
        const int r0 = kt * 32 + 16 * s + 4 * hk + jr;  // within the sub-block
#pragma unroll
        for (int dt = 0; dt < DV / 32; dt++) {
          const int col = dt * 32 + jc;
          u32x2 lo, hi;
          if constexpr (C::SWZ) {
            const int kr0 = kw * KBW + r0, kr1 = kr0 + 8;
            lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(
                Vst + r0 * ROWB + ((((col >> 3) ^ ((kr0 >> 1) & 7)) << 4) | ((col & 7) * 2))));
            hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(
                Vst + (r0 + 8) * ROWB + ((((col >> 3) ^ ((kr1 >> 1) & 7)) << 4) | ((col & 7) * 2))));
          } else {
            lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(Vst + r0 * ROWB + col * 2));
            hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(Vst + (r0 + 8) * ROWB + col * 2));
          }
          u32x4 va = {lo.x, lo.y, hi.x, hi.y};
          if (ONES && dt == DV / 32 - 1) {
            constexpr uint32_t one2 = 0x3f803f80u;  // two bf16 1.0
            va = ones_lane ? u32x4{one2, one2, one2, one2} : va;
          }
          oacc[dt] = mfma32(as_bf16x8(va), bp, oacc[dt]);
        }
      }
  }

  if constexpr (NKW > 1) {
    // ---- merge the key waves' partial results (fp32) through LDS. Only the NU registers holding output rows < D
    // are staged; every key wave finishes the groups of 4 registers (4 consecutive output rows) g with
    // g % NKW == kw, summing the partials in key-wave order
    constexpr int NU = C::NU, NW = C::NW;
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + NW * 64;
    float* co = cl + NW * 64;  // [slot][u][lane]
    wait_vm<0>();
    __syncthreads();
    const int slot = kw * NQW + qg;
    if constexpr (ONES) l_run = oacc[DV / 32 - 1][4];
    cm[slot * 64 + lane] = m_run;
    cl[slot * 64 + lane] = l_run;
#pragma unroll
    for (int u = 0; u < NU; u++) co[(slot * NU + u) * 64 + lane] = oacc[u / 16][u % 16];
    __syncthreads();
    float M = -1e30f;
#pragma unroll
    for (int k = 0; k < NKW; k++) M = fmaxf(M, cm[(k * NQW + qg) * 64 + lane]);
    float L = 0.f, f[NKW];
#pragma unroll
    for (int k = 0; k < NKW; k++) {
      f[k] = __builtin_amdgcn_exp2f(cm[(k * NQW + qg) * 64 + lane] - M);
      L += cl[(k * NQW + qg) * 64 + lane] * f[k];
    }
    if (qi >= Tq) return;
    const float inv = 1.f / L;
    uint16_t* orow = O + b * so_b + (long)qi * so_t + h * so_h;
#pragma unroll
    for (int g2 = 0; g2 < NU / 4; g2++) {
      if (g2 % NKW != kw) continue;  // wave-uniform
      float o4[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < NKW; k++) acc += co[((k * NQW + qg) * NU + 4 * g2 + u) * 64 + lane] * f[k];
        o4[u] = acc * inv;
      }
      const int dt = g2 / 4, g = g2 % 4;
      const int d = dt * 32 + 8 * g + 4 * hk;  // < D for every staged register
      u32x2 o;
      o.x = pack2(o4[0], o4[1]);
      o.y = pack2(o4[2], o4[3]);
      *reinterpret_cast<u32x2*>(orow + d) = o;
    }
    return;
  }

  if (qi >= Tq) return;
  if constexpr (ONES) l_run = oacc[DV / 32 - 1][4];
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

template <int D, int NQW, int NKW, int KB, int S>
hipError_t launch(hipStream_t st, const Args& a) {
  const long nt = (long)((a.Tq + 32 * NQW - 1) / (32 * NQW)) * a.H * a.B;
  if (nt > 0x7fffffffL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_fwd_kernel<D, NQW, NKW, KB, S>), dim3((unsigned)nt), dim3(64 * NQW * NKW), 0, st, a.Q, a.sq_b, a.sq_h,
                     a.sq_t, a.K, a.sk_b, a.sk_h, a.sk_t, a.V, a.sv_b, a.sv_h, a.sv_t, a.O, a.so_b, a.so_h, a.so_t,
                     a.Tq, a.Tk, a.H, a.H * a.B, a.sl2, a.qpos0, a.causal_from);
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

// The tiling mx_sdpa runs for a problem, from timings of every (query waves, key waves, block keys, stages) variant
// on the shapes this library runs (HIP-graph replays, us per launch on MI355X):
//  * many (batch, head, 128-query) tiles (wg4 >= 512): 4 query waves share each staged key block; with head dim 72
//    two key waves split every 64-key block as well (vision batch 13: 64.4 -> 61.6, batch 256: 1261 -> 1188);
//  * few tiles: key waves split each block so the grid still fills the GPU. 2 query waves x 4 key waves (8-wave
//    workgroups) for the vision tower at batch 1 (11.1 -> 10.6 with a warm L2; 12.6 -> 12.4 on cold buffers) and the
//    yes/no query (10.3 -> 9.9); 2 x 8 over 256-key blocks (16 waves, each block's keys in 8 slices) for TRecViT's
//    12 heads x 1280 tokens (2.062 -> 2.047 ms per streamed frame in one A/B; the same tiling made the batch-1 tower
//    slower, 2.137 -> 2.171 ms); 4 x 4 (16 waves, 128 queries) for 32 heads of many queries (text prefix
//    15.2 -> 12.9); 1 x 4 for at most 64 queries (the 64-token prompt, 8.2: larger tiles leave most of their query
//    waves empty).
// t[0..3] = query waves, key waves, keys per staged block, ring stages.
extern "C" void mx_sdpa_tiling(int B, int H, int Tq, int D, int* t) {
  const long wg4 = (long)((Tq + 127) / 128) * H * B;
  int q = 2, k = 4, kb = 128, s = 2;
  if (wg4 >= 512) {
    q = 4, k = D == 72 ? 2 : 1, kb = 64, s = D == 72 ? 4 : 3;
  } else if (Tq <= 64) {
    q = 1;
  } else if (D == 64 && wg4 >= 160) {
    q = 4;
  } else if (D == 64) {
    k = 8, kb = 256;
  }
  t[0] = q, t[1] = k, t[2] = kb, t[3] = s;
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
  int t[4];
  mx_sdpa_tiling(B, H, Tq, D, t);
  const auto is = [&](int q, int k, int kb, int s) { return t[0] == q && t[1] == k && t[2] == kb && t[3] == s; };
  hipError_t e = hipErrorInvalidValue;
  if (D == 72) {
    if (is(4, 2, 64, 4)) e = launch<72, 4, 2, 64, 4>(st, a);
    else if (is(1, 4, 128, 2)) e = launch<72, 1, 4, 128, 2>(st, a);
    else if (is(2, 4, 128, 2)) e = launch<72, 2, 4, 128, 2>(st, a);
  } else {
    if (is(4, 1, 64, 3)) e = launch<64, 4, 1, 64, 3>(st, a);
    else if (is(1, 4, 128, 2)) e = launch<64, 1, 4, 128, 2>(st, a);
    else if (is(4, 4, 128, 2)) e = launch<64, 4, 4, 128, 2>(st, a);
    else if (is(2, 4, 128, 2)) e = launch<64, 2, 4, 128, 2>(st, a);
    else if (is(2, 8, 256, 2)) e = launch<64, 2, 8, 256, 2>(st, a);
  }
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}
