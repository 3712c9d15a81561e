// bf16 GEMM with fused epilogues on gfx950 MFMA:
//   C[M,N] = epi( A[M,K] . W[N,K]^T + bias[N] )      epi = round-bf16 -> optional GELU (tanh | erf) -> optional + R
// A and W are both K-contiguous (torch Linear layout). fp32 accumulation in MFMA 32x32x16 tiles.
//
// Design (gfx950, 64-wide waves, 160 KB LDS per CU):
//  * 256-thread workgroups (4 waves) own a BM x BN tile of C; each wave owns a (BM/WGM) x (BN/WGN) sub-tile.
//  * K is walked in BK = 64 steps. Global -> register prefetch of step k+1 overlaps the MFMAs of step k; the
//    prefetched tile is stored to the other LDS buffer (double buffering, one barrier per step).
//  * LDS rows are 64 bf16 (128 B) with the 16-byte chunk index XOR-swizzled by (row & 7), so the 32 rows read by
//    one MFMA operand fetch (ds_read_b128) spread over all banks without padding.
//  * The MFMA is issued "swapped" (W as the row operand, A as the column operand), so every lane ends up with 4
//    consecutive output columns of one output row: 8-byte stores, and bias / residual read as vectors.
//  * Workgroup ids are remapped so that consecutive tiles (which share W panels) land on the same XCD and its L2.
// Rounding follows torch's bf16 Linear path: the linear output is rounded to bf16, GELU is applied to that rounded
// value and rounded again, then the residual is added in fp32 and rounded once more.
#include "common.h"

namespace {

constexpr int BK = 64;

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint16_t* __restrict__ A, long lda,
                                                        const uint16_t* __restrict__ W, long ldw,
                                                        const float* __restrict__ bias,
                                                        const uint16_t* __restrict__ R, long ldr, int r_rows,
                                                        uint16_t* __restrict__ C, long ldc,
                                                        int M, int N, int K, int act, int tiles_m, int tiles_n) {
  static_assert(WGM * WGN == 4, "4 waves per workgroup");
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int ACH = BM * BK / 8 / 256;  // 16-byte chunks per thread per stage (A)
  constexpr int WCH = BN * BK / 8 / 256;  // (W)
  static_assert(ACH >= 1 && WCH >= 1 && FM >= 1 && FN >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * BK];

  // ---- XCD-aware tile order: dispatch sends workgroup b to XCD (b % 8); give each XCD a contiguous tile range.
  const int nt = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int per = nt / 8, rem = nt % 8, xcd = b % 8, idx = b / 8;
  const int t = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int tile_m = t % tiles_m, tile_n = t / tiles_m;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int lr = lane & 31, hk = lane >> 5;

  u32x4 ra[ACH], rw[WCH];
  const u32x4 zero = {0u, 0u, 0u, 0u};

  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < ACH; j++) {
      const int i = tid + 256 * j, r = i >> 3, c = i & 7;
      const int gm = min(m0 + r, M - 1), kk = k0 + c * 8;
      ra[j] = (kk < K) ? *reinterpret_cast<const u32x4*>(A + (long)gm * lda + kk) : zero;
    }
#pragma unroll
    for (int j = 0; j < WCH; j++) {
      const int i = tid + 256 * j, r = i >> 3, c = i & 7;
      const int gn = min(n0 + r, N - 1), kk = k0 + c * 8;
      rw[j] = (kk < K) ? *reinterpret_cast<const u32x4*>(W + (long)gn * ldw + kk) : zero;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < ACH; j++) {
      const int i = tid + 256 * j, r = i >> 3, c = i & 7;
      *reinterpret_cast<u32x4*>(&As[buf][r * BK + ((c ^ (r & 7)) << 3)]) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < WCH; j++) {
      const int i = tid + 256 * j, r = i >> 3, c = i & 7;
      *reinterpret_cast<u32x4*>(&Ws[buf][r * BK + ((c ^ (r & 7)) << 3)]) = rw[j];
    }
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const int nk = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      const int c = 2 * s + hk;
      bf16x8 af[FM], wf[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int r = wm * WTM + i * 32 + lr;
        af[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&As[buf][r * BK + ((c ^ (r & 7)) << 3)]));
      }
#pragma unroll
      for (int i = 0; i < FN; i++) {
        const int r = wn * WTN + i * 32 + lr;
        wf[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&Ws[buf][r * BK + ((c ^ (r & 7)) << 3)]));
      }
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) acc[i][j] = mfma32(wf[i], af[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds output row m = .. + lr, columns n .. n+3 for each 8-row group j of the MFMA result
#pragma unroll
  for (int i = 0; i < FN; i++) {
#pragma unroll
    for (int j = 0; j < FM; j++) {
      const int m = m0 + wm * WTM + j * 32 + lr;
      if (m >= M) continue;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int n = n0 + wn * WTN + i * 32 + 8 * g + 4 * hk;
        if (n >= N) continue;
        float v[4];
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (bias) bv = *reinterpret_cast<const f32x4*>(bias + n);
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = rbf(acc[i][j][4 * g + e] + bv[e]);
        if (act == 1) {
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] = rbf(gelu_tanh(v[e]));
        } else if (act == 2) {
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] = rbf(gelu_erf(v[e]));
        }
        if (R) {
          const int rm = r_rows > 0 ? m % r_rows : m;
          const u32x2 rr = *reinterpret_cast<const u32x2*>(R + (long)rm * ldr + n);
          v[0] += lo_bf(rr.x); v[1] += hi_bf(rr.x); v[2] += lo_bf(rr.y); v[3] += hi_bf(rr.y);
        }
        u32x2 o;
        o.x = pack2(v[0], v[1]);
        o.y = pack2(v[2], v[3]);
        *reinterpret_cast<u32x2*>(C + (long)m * ldc + n) = o;
      }
    }
  }
}

struct Cfg { int bm, bn; };
constexpr Cfg kCfgs[] = {{128, 128}, {64, 128}, {128, 64}, {64, 64}, {256, 128}, {128, 256}};
constexpr int kNCfg = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int BM, int BN, int WGM, int WGN>
hipError_t launch(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
                  const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int K, int act) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WGM, WGN>), dim3(tm * tn), dim3(256), 0, st, A, lda, W, ldw, bias, R,
                     ldr, r_rows, C, ldc, M, N, K, act, tm, tn);
  return hipGetLastError();
}

}  // namespace

extern "C" int mx_gemm_ncfg(void) { return kNCfg; }

extern "C" int mx_gemm_cfg_tile(int cfg, int* bm, int* bn) {
  if (cfg < 0 || cfg >= kNCfg) return MX_EBADCFG;
  *bm = kCfgs[cfg].bm;
  *bn = kCfgs[cfg].bn;
  return MX_OK;
}

// Tile choice when the caller passes cfg < 0: minimise (rounds of workgroups over 256 CUs) x (tile work / tile
// efficiency). Larger tiles re-read less from L2 per MFMA; smaller ones fill the 256 CUs at batch-1 sizes.
extern "C" int mx_gemm_pick(int M, int N, int K) {
  static const float eff[kNCfg] = {1.0f, 0.80f, 0.80f, 0.62f, 1.08f, 1.08f};
  static const int per_cu[kNCfg] = {2, 2, 2, 2, 1, 1};
  (void)K;
  int best = 0;
  float bt = 1e30f;
  for (int c = 0; c < kNCfg; c++) {
    const long tiles = (long)((M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((N + kCfgs[c].bn - 1) / kCfgs[c].bn);
    const long slots = 256L * per_cu[c];
    const long rounds = (tiles + slots - 1) / slots;
    // a partially filled last round still costs a full tile time per CU in flight
    const float t = (float)rounds * kCfgs[c].bm * kCfgs[c].bn / eff[c] / (float)per_cu[c];
    if (t < bt) { bt = t; best = c; }
  }
  return best;
}

// Validate a GEMM call without launching (0 or a negative status). Shared by mx_gemm_bf16 and host-side tests.
extern "C" int mx_gemm_check(int cfg, const void* A, long lda, const void* W, long ldw, const void* bias,
                             const void* R, long ldr, const void* C, long ldc, int M, int N, int K, int act) {
  if (!A || !W || !C) return MX_ENULL;
  if (cfg >= kNCfg) return MX_EBADCFG;
  if (act < 0 || act > 2) return MX_EBADCFG;
  if (M < 1 || N < 1 || K < 8) return MX_ESHAPE;
  if (K % 8 || lda % 8 || ldw % 8 || lda < K || ldw < K) return MX_ESHAPE;
  if (N % 4 || ldc % 4 || ldc < N) return MX_ESHAPE;
  if (((uintptr_t)A | (uintptr_t)W) & 15) return MX_ELAYOUT;
  if ((uintptr_t)C & 7) return MX_ELAYOUT;
  if (bias && ((uintptr_t)bias & 15)) return MX_ELAYOUT;
  if (R && (((uintptr_t)R & 7) || ldr % 4 || ldr < N)) return MX_ELAYOUT;
  return MX_OK;
}

// R (optional residual) row for output row m is (r_rows > 0 ? m % r_rows : m): r_rows broadcasts one [r_rows, N]
// table (e.g. a position embedding) over a batch of stacked sequences.
extern "C" int mx_gemm_bf16(hipStream_t st, int cfg, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                            const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M,
                            int N, int K, int act) {
  const int rc = mx_gemm_check(cfg, A, lda, W, ldw, bias, R, ldr, C, ldc, M, N, K, act);
  if (rc) return rc;
  if (r_rows < 0) return MX_ESHAPE;
  if (cfg < 0) cfg = mx_gemm_pick(M, N, K);
  hipError_t e;
  switch (cfg) {
    case 0: e = launch<128, 128, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    case 1: e = launch<64, 128, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    case 2: e = launch<128, 64, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    case 3: e = launch<64, 64, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    case 4: e = launch<256, 128, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    case 5: e = launch<128, 256, 2, 2>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, act); break;
    default: return MX_EBADCFG;
  }
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}
