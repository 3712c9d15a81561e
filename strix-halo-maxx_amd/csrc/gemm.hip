// bf16 GEMM with fused epilogues on gfx950 MFMA:
//   C[M,N] = epi( A[M,K] . W[N,K]^T + bias[N] )      epi = round-bf16 -> optional GELU (tanh | erf) -> optional + R
// A and W are K-contiguous (torch Linear layout); fp32 accumulation in MFMA 32x32x16 tiles.
//
// Design (gfx950: 64-wide waves, 160 KB LDS per CU, 256 CUs in 8 XCDs):
//  * 256-thread workgroups (4 waves) own a BM x BN tile of C; each wave owns a (BM/WGM) x (BN/WGN) sub-tile.
//  * Operands go global -> LDS with the asynchronous LDS-DMA load (global_load_lds_dwordx4: 64 lanes x 16 B land
//    as 1 KB in LDS without passing through VGPRs), into an S-stage LDS ring, S-1 k-steps ahead of the MFMAs.
//    The compiler cannot see which ring slot an LDS read touches, so these loads are issued from inline asm and the
//    wait for "stage k has landed" is an explicit `s_waitcnt vmcnt(n)` that leaves the later stages in flight.
//  * LDS rows are 64 bf16 (128 B) with the 16-byte chunk index XOR-swizzled by ((row >> 1) & 7): a ds_read_b128
//    serves 16 lanes (256 B, two rows per bank sweep of the 64 banks) at a time, and the 16 rows those lanes read
//    then cover every (row parity, chunk) pair once. The DMA lane -> address map is fixed (lane l writes bytes
//    16 l.. of a 1 KB block of 8 rows), so each lane fetches the global chunk that belongs at its slot; for rows
//    8 g + (l >> 3) the swizzle is (l >> 4) | ((g & 1) << 2), and g & 1 is the wave's parity.
//  * The MFMA is issued "swapped" (W as the row operand, A as the column operand): every lane ends up with 4
//    consecutive output columns of one output row -> 8-byte stores; bias / residual are read as vectors.
//  * Split-K for small grids (batch-1 shapes on 256 CUs): each split writes an fp32 partial tile; the last split to
//    arrive (atomic counter per tile) adds the partials in split order (deterministic) and runs the epilogue, then
//    re-arms the counter. No workgroup ever waits on another.
//  * Workgroup ids are remapped so consecutive tiles (sharing W panels) land on the same XCD and its L2.
//  * A second kernel kind for grids that cannot put several workgroups on every CU (batch-1 shapes), where one wave
//    per SIMD has nothing to hide the ds_read -> MFMA chain of a k-step behind: the same LDS ring, but the waves
//    split each 64-wide k-step instead of the tile. Wave w multiplies k columns [16 w, 16 w + 16) into its own copy
//    of the whole BM x BN tile, so its (BM / 32) x (BN / 32) MFMAs per k-step are independent and each LDS byte is
//    read by one wave only; the four partial tiles are summed through LDS in a fixed order after the k loop.
// Rounding follows torch's bf16 Linear path: the linear output is rounded to bf16, GELU is applied to that rounded
// value and rounded again, then the residual is added in fp32 and rounded once more.
//
// Operand contract: A has K valid columns; the k loop runs to Kw (a multiple of 64, >= K) and W must hold zeros in
// columns [K, Kw). A chunks beyond K are fetched from column 0 of the same row (finite data times W's zeros).
#include <mutex>

#include "common.h"

namespace {

constexpr int BK = 64;

// Tile order. Dispatch sends workgroup b to XCD (b % 8), so each XCD is given a contiguous run of the tile sequence
// (split-major, then tile). Inside a run, tiles go in groups of GM row panels, column-major within a group: the 32
// workgroups an XCD runs at once then share GM panels of A and a few panels of W in that XCD's L2, instead of
// sweeping every row panel of A past one W panel. Grids with at most GM row panels keep plain column-major order.
// GM = 8, and 4 for the 192- and 256-row tiles of large grids (1-3 % faster there than 8; 16 and 32 were slower).
template <int GM = 8>
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int splits, int& tm, int& tn, int& split) {
  const int nt = tiles_m * tiles_n, ntot = nt * splits;
  const int per = ntot / 8, rem = ntot % 8, xcd = b % 8, idx = b / 8;
  const int t = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int tile = t % nt;
  split = t / nt;
  const int grp = tile / (GM * tiles_n), first = grp * GM, gs = min(tiles_m - first, GM);
  const int r = tile - grp * GM * tiles_n;
  tm = first + r % gs;
  tn = r / gs;
}

// Epilogue of one 4-column group (output row m, columns n .. n+3) from fp32 sums s: + bias, round to bf16, activation
// ACT (1 GELU-tanh, 2 GELU-erf; rounded again; skipped for columns >= act_ncols when act_ncols > 0), + residual
// (fp32 add, rounded once more). ACT 3 is the gated GELU of interleaved (gate, up) column pairs, written to columns
// n / 2, n / 2 + 1.
template <int V>
struct IntC {
  static constexpr int value = V;
};
// I8: s holds int32 accumulator bits; the linear output is ((float)acc * sa) * sw + bias in fp32 and any GELU applies
// to that fp32 value before the one bf16 rounding (the W8A8 epilogue); a residual is then added to the rounded value.
// HR: 0 / 1 = no residual / a residual, known at compile time; 2 = has_r decides. The activation is computed for every
// column and then selected (act_ncols varies across the lanes of a wave: a branch per group would serialise the
// exp / rcp chains of the groups instead of interleaving them).
template <int ACT, bool I8 = false, int HR = 2>
__device__ __forceinline__ u32x2 epi_val(const f32x4& s, const f32x4& bv, const u32x2& rv, bool has_r, int n,
                                         int act_ncols, float sa = 0.f, const f32x4& sw = f32x4{0.f, 0.f, 0.f, 0.f}) {
  const bool hr = HR == 2 ? has_r : HR == 1;
  float v[4];
  if constexpr (I8) {
    static_assert(ACT != 3, "no gated GELU in the int8 path");
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float t = (float)__float_as_int(s[e]) * sa;
      v[e] = t * sw[e] + bv[e];
    }
    if constexpr (ACT == 1 || ACT == 2) {
      const bool on = act_ncols <= 0 || n < act_ncols;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float g = ACT == 1 ? gelu_tanh(v[e]) : gelu_erf(v[e]);
        v[e] = on ? g : v[e];
      }
    }
    if (hr) {
      v[0] = rbf(v[0]) + lo_bf(rv.x);
      v[1] = rbf(v[1]) + hi_bf(rv.x);
      v[2] = rbf(v[2]) + lo_bf(rv.y);
      v[3] = rbf(v[3]) + hi_bf(rv.y);
    }
    return u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
  }
#pragma unroll
  for (int e = 0; e < 4; e++) v[e] = rbf(s[e] + bv[e]);
  u32x2 o;
  if constexpr (ACT == 3) {
    o.x = pack2(rbf(gelu_tanh(v[0])) * v[1], rbf(gelu_tanh(v[2])) * v[3]);
    o.y = 0;
  } else {
    if constexpr (ACT == 1 || ACT == 2) {
      // the activation's bf16 rounding: explicit before a residual add, else the final pack's own rounding
      const bool on = act_ncols <= 0 || n < act_ncols;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float g = ACT == 1 ? gelu_tanh(v[e]) : gelu_erf(v[e]);
        if (hr) g = rbf(g);
        v[e] = on ? g : v[e];
      }
    }
    if (hr) {
      v[0] += lo_bf(rv.x);
      v[1] += hi_bf(rv.x);
      v[2] += lo_bf(rv.y);
      v[3] += hi_bf(rv.y);
    }
    o.x = pack2(v[0], v[1]);
    o.y = pack2(v[2], v[3]);
  }
  return o;
}
// Group result into the LDS staging tile (row pitch SP elements) at tile row r, tile column c (ACT 3: column c / 2).
template <int ACT, int SP>
__device__ __forceinline__ void stage_val(uint16_t* st, int r, int c, const u32x2& o) {
  if constexpr (ACT == 3)
    *reinterpret_cast<uint32_t*>(st + r * SP + (c >> 1)) = o.x;
  else
    *reinterpret_cast<u32x2*>(st + r * SP + c) = o;
}
// Staged ROWS x COLS tile (LDS, row pitch PITCH elements of T) -> C[m0 + r][c0 + c], rows < M, columns < Ncols.
// The workgroup's 256 threads take consecutive 16-byte chunks of consecutive rows, so each wave store covers whole
// cache lines (the MFMA layout alone would write 16-32 bytes into each of 32 lines per store).
template <int ROWS, int COLS, int PITCH, int NT = 256, typename T>
__device__ __forceinline__ void store_staged(const T* st, T* __restrict__ C, long ldc, int m0, int c0, int M, int Ncols,
                                             int tid) {
  constexpr int EPC = 16 / sizeof(T), CPR = (COLS + EPC - 1) / EPC, TOT = ROWS * CPR;
  const bool a16 = ((ldc * (long)sizeof(T)) % 16 == 0) && ((uintptr_t)C % 16 == 0) && ((c0 * (int)sizeof(T)) % 16 == 0);
#pragma unroll
  for (int idx0 = 0; idx0 < TOT; idx0 += NT) {
    const int idx = idx0 + tid;
    if (idx < TOT) {
      const int r = idx / CPR, cc = idx % CPR;
      const int m = m0 + r, n = c0 + cc * EPC;
      if (m < M && n < Ncols) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * PITCH + cc * EPC);
        T* dst = C + (long)m * ldc + n;
        if (n + EPC <= Ncols && a16) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else {  // unaligned row or the row's tail: 4-byte words (callers keep rows 4-byte aligned)
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
          const int nw = min(4, (Ncols - n) * (int)sizeof(T) / 4);
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (e < nw) reinterpret_cast<uint32_t*>(dst)[e] = w[e];
        }
      }
    }
  }
}
// Group operands, read from clamped (always valid) addresses; values of out-of-range groups are never stored.
__device__ __forceinline__ f32x4 bias4(const float* __restrict__ bias, int n, int N) {
  return *reinterpret_cast<const f32x4*>(bias + min(n, N - 4));
}
__device__ __forceinline__ u32x2 res4(const uint16_t* __restrict__ R, long ldr, int r_rows, int m, int n, int M, int N) {
  int rm = min(m, M - 1);
  if (r_rows > 0) rm %= r_rows;
  return *reinterpret_cast<const u32x2*>(R + (long)rm * ldr + min(n, N - 4));
}
// Run f(IntC<act>) for the runtime activation code act (0..3).
template <typename F>
__device__ __forceinline__ void with_act(int act, F&& f) {
  switch (act) {
    case 1: f(IntC<1>{}); break;
    case 2: f(IntC<2>{}); break;
    case 3: f(IntC<3>{}); break;
    default: f(IntC<0>{}); break;
  }
}

// Scheduling groups for one substep of the software pipeline: R LDS reads (of the next substep's fragments), each
// followed by its share of the F MFMAs (of this substep), so the reads are spread under the matrix work.
template <int R, int F, int r = 0>
__device__ __forceinline__ void interleave_reads_mfma() {
  if constexpr (r < R) {
    constexpr int n = F * (r + 1) / R - F * r / R;
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x008, n, 0);  // then n MFMAs
    interleave_reads_mfma<R, F, r + 1>();
  }
}

// ---- fused residual + LayerNorm epilogue (mx_gemm_bf16_res_ln): x' = bf16(bf16(acc + bias) + R) and Y = LN(x').
// A row's LayerNorm needs all N columns, which tiles_n workgroups hold. Each publishes, for each of its BM rows, the
// sum of its BN values of x' and their centred square sum as two 64-bit words (epoch << 32 | fp32 bits), written
// with single-copy-atomic agent-scope stores and read with agent-scope loads (past the per-XCD L2s), and waits only
// for the other tiles of its row block. The epoch is the row block's generation + 1; the generation lives in device
// memory, every workgroup reads it after its k loop, and the row block's first column tile writes the epoch back as
// the generation once it has seen all of the row block's words, so every launch (graph replays included) uses new
// epochs and nothing is ever cleared. The waits are bounded (kRlnTimeout); a timeout sets sync[0] and the
// launch's results are garbage. Every workgroup of a row block must be resident at once: the host allows this mode
// only for grids of at most one workgroup per CU.
struct RlnArgs {
  const uint16_t* gamma;
  const uint16_t* beta;
  uint16_t* X;   // x' (ldx)
  long ldx;
  uint16_t* Y;   // LN(x') (ldy)
  long ldy;
  float eps;
  uint64_t* stats;  // [tiles_m][tiles_n][BM][2] words
  uint32_t* sync;   // [0] error word, then the generation of each row block
};
constexpr uint64_t kRlnTimeout = 5000000ull;  // 50 ms at 100 MHz (s_memrealtime)
constexpr int kRlnMaxTiles = 64;             // column tiles per row (N <= 64 BN)
#define GPTR(T, p) ((__attribute__((address_space(1))) T*)(p))

// The kernel body, shared by the bf16 GEMM and the W8A8 int8 GEMM (I8). In the int8 form A and W hold int8 values and
// every K / stride argument counts 16-bit units (2 int8): an LDS row is still 128 bytes (128 int8 of one k-step), a
// fragment is still 16 bytes (16 consecutive k for the 32x32x32 int8 MFMA instead of 8 for the 32x32x16 bf16 one), so
// the DMA, swizzle and pipeline are unchanged; the accumulators hold int32 bits.
// KS = 2: 8 waves, the spatial WGM x WGN split twice over, each wave group taking half of every k-step's substeps
// (same LDS bytes per k-step as KS = 1, twice the waves to pull them: a CU holding one workgroup reads its LDS at the
// 8-wave rate); the second group's accumulators are added to the first's through LDS after the k loop.
template <int BM, int BN, int WGM, int WGN, int S, bool I8, int KS = 1, int RLN = 0>
__device__ __forceinline__ void gemm_body(
    const uint16_t* __restrict__ A, long lda, const uint16_t* __restrict__ W, long ldw,
    const float* __restrict__ bias, const uint16_t* __restrict__ R, long ldr, int r_rows,
    uint16_t* __restrict__ C, long ldc, int M, int N, int K, int Kw, int act, int act_ncols,
    int tiles_m, int tiles_n, int splits, int kt_per_split, float* __restrict__ ws, int* __restrict__ cnt,
    float* __restrict__ P, long ldp, long p_split, const float* __restrict__ sa, const float* __restrict__ sw,
    const RlnArgs rl = RlnArgs{}) {
  constexpr int NWS = WGM * WGN, NW = NWS * KS, NT = 64 * NW;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves per workgroup");
  static_assert(KS == 1 || KS == 2, "one or two k groups");
  constexpr int SPW = (BK / 16) / KS;  // 16-wide substeps per wave per k-step
  static_assert(S >= 2, "at least a double buffer");
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int QA = BM / (8 * NW), QW = BN / (8 * NW);  // DMA instructions per wave per stage
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "whole DMA instructions per wave");
  constexpr int LPS = QA + QW;
  constexpr int STAGE = (BM + BN) * BK;      // elements per ring stage
  static_assert(FM >= 1 && FN >= 1 && QA >= 1 && QW >= 1, "tile too small");
  constexpr int SP = BN + 8;  // row pitch of the epilogue's staging tile (reuses the ring)
  constexpr int SPF = BN + 4;  // row pitch of the fp32 staging tile of the partial-sum mode (4-wave tiles)
  constexpr int SMEM0 = S * STAGE > BM * SP ? S * STAGE : BM * SP;
  // partial-sum mode: 2 x 2 spatial tiles whose fp32 staging tile fits the LDS; in-kernel split-K only without KS
  constexpr bool PSUM = NWS == 4 && BM * BN <= 128 * 256;
  constexpr int SMEM = PSUM && BM * SPF * 2 > SMEM0 ? BM * SPF * 2 : SMEM0;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[SMEM];

  // large tiles: row groups of 4, and the refill of the ring interleaved with the last substep's MFMAs (below)
  constexpr bool BIG = BM * BN >= 192 * 192;
  int tile_m, tile_n, split;
  tile_of<BIG ? 4 : 8>(blockIdx.x, tiles_m, tiles_n, splits, tile_m, tile_n, split);
  const int tile = tile_n * tiles_m + tile_m;  // split-K workspace slot
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int nk_all = Kw / BK;
  const int kt0 = split * kt_per_split;
  const int nkl = min(nk_all, kt0 + kt_per_split) - kt0;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wsp = wave % NWS, kh = wave / NWS;  // spatial wave, k group
  const int wm = wsp % WGM, wn = wsp / WGM;
  const bool owner = kh == 0;                   // holds the summed tile after the k loop
  const int lr = lane & 31, hk = lane >> 5;
  const uint32_t sbase = lds_off(smem);

  // per-lane DMA source rows / chunk (fixed for the whole k loop)
  const int drow = lane >> 3, dch = (lane & 7) ^ ((lane >> 4) | ((wave & 1) << 2));
  const uint16_t* a_src[QA];
  const uint16_t* w_src[QW];
#pragma unroll
  for (int q = 0; q < QA; q++) {
    const int gm = min(m0 + 8 * (q * NW + wave) + drow, M - 1);
    a_src[q] = A + (long)gm * lda;
  }
#pragma unroll
  for (int q = 0; q < QW; q++) {
    const int gn = min(n0 + 8 * (q * NW + wave) + drow, N - 1);
    w_src[q] = W + (long)gn * ldw;
  }
  auto issue = [&](int kt, int s) {
    const int kk = kt * BK + dch * 8;
    const int ka = kk < K ? kk : 0;
    const uint32_t st = sbase + (uint32_t)(s * STAGE * 2);
#pragma unroll
    for (int q = 0; q < QA; q++) dma16(a_src[q] + ka, __builtin_amdgcn_readfirstlane(st + (q * NW + wave) * 1024));
#pragma unroll
    for (int q = 0; q < QW; q++)
      dma16(w_src[q] + kk, __builtin_amdgcn_readfirstlane(st + BM * 128 + (q * NW + wave) * 1024));
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // Software pipeline. Operand fragments are double-buffered in registers: while the MFMAs of 16-wide substep s
  // run, the LDS reads of substep s + 1 are in flight (one read between every few MFMAs). The ring slot of k-step it
  // is refilled (stage it + S) right after the barrier that ends its last reads, and that barrier, the refill and the
  // first reads of k-step it + 1 all sit under the MFMAs of k-step it's last substep. So the prologue fills all S
  // slots and S - 1 stages stay in flight behind the one being consumed.
  bf16x8 af[2][FM], wf[2][FN];
  auto read_frags = [&](int buf, const uint16_t* As, int s) {
    const uint16_t* Ws = As + BM * BK;
    const int c = 2 * s + hk;
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int r = wm * WTM + i * 32 + lr;
      af[buf][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&As[r * BK + ((c ^ ((r >> 1) & 7)) << 3)]));
    }
#pragma unroll
    for (int i = 0; i < FN; i++) {
      const int r = wn * WTN + i * 32 + lr;
      wf[buf][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&Ws[r * BK + ((c ^ ((r >> 1) & 7)) << 3)]));
    }
  };
  auto mfma1 = [&](int buf, int i, int j) {
    if constexpr (I8) {
      typedef int i32x4 __attribute__((ext_vector_type(4)));
      typedef int i32x16 __attribute__((ext_vector_type(16)));
      acc[i][j] = __builtin_bit_cast(f32x16, __builtin_amdgcn_mfma_i32_32x32x32_i8(
          __builtin_bit_cast(i32x4, wf[buf][i]), __builtin_bit_cast(i32x4, af[buf][j]),
          __builtin_bit_cast(i32x16, acc[i][j]), 0, 0, 0));
    } else {
      acc[i][j] = mfma32(wf[buf][i], af[buf][j], acc[i][j]);
    }
  };
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++) mfma1(buf, i, j);
  };
  // interleave the FM + FN reads of the next substep with the FM * FN MFMAs of this one
  auto interleave = [&]() {
#ifndef GEMM_NO_INTERLEAVE
    interleave_reads_mfma<FM + FN, FM * FN>();
#endif
  };

  // The epilogue's operands: bias, per-row / per-column scales and, on 4-wave tiles, the residual. Small 4-wave tiles
  // load them before the k loop, so their latency hides under it (nothing in the loop uses them, so the compiler puts
  // no wait for them there); larger tiles load them after it (their registers are taken). Each
  // pointer is checked: the raw-sum modes (P) return before the epilogue and may pass null scales, bias or residual.
  constexpr bool HOIST_R = FN * FM <= 4;
  // 2 x 2 blocks per wave hold 47 more VGPRs through the loop: only where the ring already keeps the CU to one
  // workgroup (more than 80 KB of LDS); with a smaller ring they would halve the workgroups per CU (> 256 registers)
  constexpr bool EARLY = NW == 4 && (FN * FM <= 2 || (FN * FM <= 4 && S * STAGE * 2 > 80 * 1024));
  f32x4 bv[FN][4];
  f32x4 swv[I8 ? FN : 1][4];
  float sav[I8 ? FM : 1];
  u32x2 rv[HOIST_R ? FN : 1][HOIST_R ? FM : 1][4];
  // RLN: 0 plain epilogue, 1 residual + LayerNorm (gamma, beta), 2 residual + RMSNorm (gamma = sc1, no beta)
  constexpr bool RMS = RLN == 2;
  u32x2 gmv[RLN ? FN : 1][4], btv[RLN ? FN : 1][4];
  if constexpr (RLN) {
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int c = n0 + wn * WTN + i * 32 + 8 * g + 4 * hk;  // < N: N is a multiple of BN in this mode
        gmv[i][g] = *reinterpret_cast<const u32x2*>(rl.gamma + c);
        btv[i][g] = RMS ? u32x2{0u, 0u} : *reinterpret_cast<const u32x2*>(rl.beta + c);
      }
  }
  if constexpr (EARLY) {
    if constexpr (I8) {
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          swv[i][g] = sw ? bias4(sw, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, N) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < FM; j++) sav[j] = sa ? sa[min(m0 + wm * WTM + j * 32 + lr, M - 1)] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        bv[i][g] = bias ? bias4(bias, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, N) : f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (HOIST_R) {
      if (R) {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
          for (int j = 0; j < FM; j++)
#pragma unroll
            for (int g = 0; g < 4; g++)
              rv[i][j][g] = res4(R, ldr, r_rows, m0 + wm * WTM + j * 32 + lr, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, M, N);
      }
    }
  }
#pragma unroll
  for (int s = 0; s < S; s++)
    if (s < nkl) issue(kt0 + s, s);
  wait_stages<LPS, S - 1>(nkl - 1);  // stage 0 has landed
  __syncthreads();
  read_frags(0, smem, kh * SPW);

  for (int it = 0; it < nkl; it++) {
    const uint16_t* As = smem + (it % S) * STAGE;
#pragma unroll
    for (int s = 0; s < SPW - 1; s++) {
      read_frags((s + 1) & 1, As, kh * SPW + s + 1);
      mfmas(s & 1);
      interleave();
    }
    __builtin_amdgcn_sched_barrier(0);
    // stage it + 1 has landed once at most (stages issued after it) x LPS loads are still in flight; the barrier
    // also ends every wave's reads of slot it % S, which is refilled with stage it + S. On the last k-step nothing is
    // in flight and the reads below fetch a stale slot that is never used: one copy of the MFMAs, no branch around
    // them (two copies would make the register allocator keep two accumulator sets).
    wait_stages<LPS, S - 2>(nkl - 2 - it);
    __syncthreads();
    if constexpr (BIG) {
      // the next substep's reads first (the DMA's memory clobber would hold them back), then one DMA instruction of
      // stage it + S after each MFMA of the last substep, so the MFMA pipe is not idle while the refill issues
      read_frags(0, smem + ((it + 1) % S) * STAGE, kh * SPW);
      const bool refill = it + S < nkl;
      const int kk = (kt0 + it + S) * BK + dch * 8;
      const int ka = kk < K ? kk : 0;
      const uint32_t st = sbase + (uint32_t)((it % S) * STAGE * 2);
      auto one = [&](int t) {  // t is a constant after unrolling
        if (t < QA)
          dma16(a_src[t < QA ? t : 0] + ka, __builtin_amdgcn_readfirstlane(st + (t * NW + wave) * 1024));
        else
          dma16(w_src[t >= QA && t - QA < QW ? t - QA : 0] + kk,
                __builtin_amdgcn_readfirstlane(st + BM * 128 + ((t - QA) * NW + wave) * 1024));
      };
      constexpr int buf = (SPW - 1) & 1;
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) {
          mfma1(buf, i, j);
          const int t = i * FM + j;
          if (t < LPS) {
            __builtin_amdgcn_sched_barrier(0);
            if (refill) one(t);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
#pragma unroll
      for (int t = FN * FM; t < LPS; t++)
        if (refill) one(t);
    } else {
      if (it + S < nkl) issue(kt0 + it + S, it % S);
      read_frags(0, smem + ((it + 1) % S) * STAGE, kh * SPW);
      mfmas((SPW - 1) & 1);
      interleave();
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  static_assert(SPW % 2 == 0, "the tail reads into buffer 0");

  if constexpr (RLN) {
    static_assert(KS == 1 && !I8 && NWS == 4 && WGN == 2 && EARLY && HOIST_R, "4-wave 2 x 2 tiles, small");
    static_assert(NT % BM == 0 && BM <= NT, "whole row groups of threads");
    constexpr int QG = NT / BM;  // thread groups per row when the statistics are gathered
    const int rb = tile_m;
    uint32_t* gen = rl.sync + 1 + rb;
    // every workgroup of the row block reads the generation before it publishes; none advances it before all have
    // published, so all of them use the same epoch. (Read here, its round trip hides under the statistics below; read
    // before the k loop, the loads of 216 workgroups at one address held up the ring's first loads: 2.31 against
    // 2.19 ms per frame.)
    const uint32_t ep = __hip_atomic_load(GPTR(uint32_t, gen), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    // x' in registers: bf16(bf16(acc + bias) + residual), the rounding of residual_layernorm_kernel
    float xv[FN][FM][16];
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float r4[4] = {lo_bf(rv[i][j][g].x), hi_bf(rv[i][j][g].x), lo_bf(rv[i][j][g].y), hi_bf(rv[i][j][g].y)};
#pragma unroll
          for (int e = 0; e < 4; e++) xv[i][j][4 * g + e] = rbf(rbf(acc[i][j][4 * g + e] + bv[i][g][e]) + r4[e]);
        }
    float* red = reinterpret_cast<float*>(smem);  // [QG][BM] partials (the ring is free past the k loop)
    float* red2 = red + QG * BM;
    float* smean = red2 + QG * BM;                // [BM] mean, [BM] rstd
    float* srstd = smean + BM;
    uint16_t* stx = reinterpret_cast<uint16_t*>(srstd + BM);  // staging tile of x', then of Y (BM x SP)
    static_assert((4 * QG * BM + 2 * BM) * 4 + BM * SP * 2 <= SMEM * 2, "the epilogue fits the ring");
    // this tile's row sums, then centred square sums (two passes over registers, waves wn = 0, 1 combined in order);
    // RMSNorm: the row sums of bf16(x'^2) only
    float tsum[FM], tm2[FM];
    __syncthreads();  // every wave is past its last ring read
#pragma unroll
    for (int j = 0; j < FM; j++) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) a += RMS ? rbf(xv[i][j][e] * xv[i][j][e]) : xv[i][j][e];
      a = halves_sum(a);
      if (hk == 0) red[wn * BM + wm * WTM + j * 32 + lr] = a;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FM; j++) {
      const int r = wm * WTM + j * 32 + lr;
      tsum[j] = red[r] + red[BM + r];
      if constexpr (RMS) continue;
      const float mt = tsum[j] * (1.0f / BN);
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const float d = xv[i][j][e] - mt;
          q += d * d;
        }
      q = halves_sum(q);
      if (hk == 0) red2[wn * BM + r] = q;
    }
    // x' to the staging tile meanwhile
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int r = wm * WTM + j * 32 + lr, c = wn * WTN + i * 32 + 8 * g + 4 * hk;
          *reinterpret_cast<u32x2*>(stx + r * SP + c) =
              u32x2{pack2(xv[i][j][4 * g], xv[i][j][4 * g + 1]), pack2(xv[i][j][4 * g + 2], xv[i][j][4 * g + 3])};
        }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FM; j++) tm2[j] = RMS ? 0.f : red2[wm * WTM + j * 32 + lr] + red2[BM + wm * WTM + j * 32 + lr];
    // publish (one lane per row: the wn = 0, hk = 0 lanes)
    uint64_t* sbase = rl.stats + ((size_t)rb * tiles_n) * BM * 2;
    if (wn == 0 && hk == 0) {
#pragma unroll
      for (int j = 0; j < FM; j++) {
        const int r = wm * WTM + j * 32 + lr;
        uint64_t* w = sbase + ((size_t)tile_n * BM + r) * 2;
        __hip_atomic_store(GPTR(uint64_t, w), ((uint64_t)ep << 32) | __float_as_uint(tsum[j]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(GPTR(uint64_t, w + 1), ((uint64_t)ep << 32) | __float_as_uint(tm2[j]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // x' out while the other tiles publish
    store_staged<BM, BN, SP, NT>(stx, rl.X, rl.ldx, m0, n0, M, N, tid);
    // gather: thread (q, r) reads the entries of tiles q, q + QG, ... for row r, until all carry this epoch
    {
      const int r = tid % BM, q = tid / BM;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(sbase, (short)0, (int)(tiles_n * BM * 16), 0x00020000);
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      float ssum = 0.f;
      constexpr int KMAX = (kRlnMaxTiles + QG - 1) / QG;
      float es[KMAX], em2[KMAX];  // fixed indices only (unrolled, predicated): registers, not scratch
      const int nmine = (tiles_n - q + QG - 1) / QG;
      for (;;) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < KMAX; k++) {
          es[k] = 0.f;
          em2[k] = 0.f;
          if (k < nmine) {
            uint32_t off = (uint32_t)(((q + k * QG) * BM + r) * 16);
            asm volatile("" : "+v"(off));  // a new offset each pass: the load is not hoisted out of the loop
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 16);
            ok = ok && v.y == ep && v.w == ep;
            es[k] = __uint_as_float(v.x);
            em2[k] = __uint_as_float(v.z);
          }
        }
        if (ok) break;
        if (__builtin_amdgcn_s_memrealtime() - t0 > kRlnTimeout) {
          __hip_atomic_store(GPTR(uint32_t, rl.sync), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int k = 0; k < KMAX; k++) ssum += es[k];  // zeros past nmine
      red[q * BM + r] = ssum;
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < QG; k2++) tot += red[k2 * BM + r];
      if constexpr (RMS) {  // rstd = bf16(1 / sqrt(bf16(bf16(sum / N) + eps))), the rounding of rmsnorm_kernel
        if (q == 0) {
          smean[r] = 0.f;
          srstd[r] = rbf(1.0f / sqrtf(rbf(rbf(tot / (float)N) + rl.eps)));
        }
      }
      const float mean = tot / (float)N;
      // M2 = sum over tiles of (M2_t + BN (mean_t - mean)^2): the centred square sum over the whole row
      float m2 = 0.f;
#pragma unroll
      for (int k = 0; k < KMAX; k++) {
        const float d = es[k] * (1.0f / BN) - mean;
        m2 += k < nmine ? em2[k] + (float)BN * d * d : 0.f;
      }
      red2[q * BM + r] = m2;
      __syncthreads();
      if (!RMS && q == 0) {
        float t2 = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < QG; k2++) t2 += red2[k2 * BM + r];
        smean[r] = mean;
        srstd[r] = 1.0f / sqrtf(t2 / (float)N + rl.eps);
      }
    }
    __syncthreads();  // statistics read by every thread of this workgroup; the staging tile of x' is stored
    // every tile of the row block has published this epoch (so every workgroup of it has read the generation): the
    // row block's first column tile writes it as the next launch's generation. (No departure counter, whose returning
    // atomic held every wave at the barrier before the Y store; and one writer per row block: 216 agent-scope stores
    // into one cache line, one per workgroup, made the tower 2.33 against 2.21 ms per frame.)
    if (tid == 0 && tile_n == 0) __hip_atomic_store(GPTR(uint32_t, gen), ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Y = (x' - mean) rstd gamma + beta, the order of residual_layernorm_kernel
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++) {
        const int r = wm * WTM + j * 32 + lr;
        const float mu = smean[r], rs2 = srstd[r];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float gg[4] = {lo_bf(gmv[i][g].x), hi_bf(gmv[i][g].x), lo_bf(gmv[i][g].y), hi_bf(gmv[i][g].y)};
          const float bb[4] = {lo_bf(btv[i][g].x), hi_bf(btv[i][g].x), lo_bf(btv[i][g].y), hi_bf(btv[i][g].y)};
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; e++)
            y[e] = RMS ? rbf(xv[i][j][4 * g + e] * rs2) * gg[e] : (xv[i][j][4 * g + e] - mu) * rs2 * gg[e] + bb[e];
          const int c = wn * WTN + i * 32 + 8 * g + 4 * hk;
          *reinterpret_cast<u32x2*>(stx + r * SP + c) = u32x2{pack2(y[0], y[1]), pack2(y[2], y[3])};
        }
      }
    __syncthreads();
    store_staged<BM, BN, SP, NT>(stx, rl.Y, rl.ldy, m0, n0, M, N, tid);
    return;
  }

  // ---- KS = 2: the second k group's partial tiles join the first's, in a fixed order. The first group finishes
  // every accumulator block, except in the partial-sum mode, where each group finishes every other block (sums
  // and fp32 staging split over all 8 waves; the same bits, fp32 addition being commutative). Measured in context:
  // TRecViT's 2-split partials 1.923-1.925 -> 1.909-1.912 ms per streamed frame, the tower unchanged; the same split
  // of the bias / GELU epilogue made the batch-1 tower 0.8 % slower.
  const bool split_epi = KS == 2 && (FN * FM) % 2 == 0 && PSUM && P != nullptr;
  auto mine = [&](int i, int j) { return split_epi ? ((i * FM + j) & 1) == kh : owner; };
  if constexpr (KS == 2) {
    float* red = reinterpret_cast<float*>(smem);
    static_assert(NWS * FN * FM * 16 * 64 * 4 <= S * STAGE * 2, "the exchange fits the ring");
    __syncthreads();  // every wave is past its last ring read
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
        if (!mine(i, j)) {
#pragma unroll
          for (int e = 0; e < 16; e++) red[(((wsp * FN + i) * FM + j) * 16 + e) * 64 + lane] = acc[i][j][e];
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
        if (mine(i, j)) {
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const float o = red[(((wsp * FN + i) * FM + j) * 16 + e) * 64 + lane];
            if constexpr (I8)
              acc[i][j][e] = __int_as_float(__float_as_int(acc[i][j][e]) + __float_as_int(o));
            else
              acc[i][j][e] += o;
          }
        }
  }

  // ---- partial-sum mode (mx_gemm_bf16_partial): this split's raw fp32 sums to its slab of P, staged like the bf16
  // results; no bias, activation or residual
  if constexpr (PSUM) {
    if (P) {
      float* stf = reinterpret_cast<float*>(smem);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++)
          if (mine(i, j)) {
#pragma unroll
            for (int g = 0; g < 4; g++)
              *reinterpret_cast<f32x4*>(stf + (wm * WTM + j * 32 + lr) * SPF + wn * WTN + i * 32 + 8 * g + 4 * hk) =
                  f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          }
      __syncthreads();
      store_staged<BM, BN, SPF, NT>(stf, P + split * p_split, ldp, m0, n0, M, N, tid);
      return;
    }
  }

  // ---- split-K: partial tile to the workspace; the last split to arrive reduces in split order (4-wave tiles only:
  // the 8-wave tiles serve grids large enough without it)
  if (PSUM && KS == 1 && !I8 && splits > 1) {
    constexpr int TE = BM * BN;
    float* mine = ws + (long)(tile * splits + split) * TE;
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) mine[(((wave * FN + i) * FM + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    __threadfence();
    __syncthreads();
    // the arrival flag lives in the ring's last 4 bytes: every wave is past its last LDS read here
    int* s_last = reinterpret_cast<int*>(smem + SMEM - 2);
    if (tid == 0) *s_last = (atomicAdd(&cnt[tile], 1) == splits - 1);
    __syncthreads();
    if (!*s_last) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const long o = (((wave * FN + i) * FM + j) * 16 + e) * 64 + lane;
          float v = 0.f;
          for (int s = 0; s < splits; s++) {
            const float p = (s == split) ? acc[i][j][e] : __builtin_nontemporal_load(ws + (long)(tile * splits + s) * TE + o);
            v = (s == 0) ? p : v + p;
          }
          acc[i][j][e] = v;
        }
    if (tid == 0) cnt[tile] = 0;
  }

  // ---- epilogue: lane holds output row m, columns n .. n+3 for each 8-row group g of the MFMA result. Results go
  // through an LDS staging tile (the ring is free once every wave is past its last k-step) and reach C only in the
  // final copy. The bias, scales and residual were loaded before the k loop (small tiles) or are loaded here.
  if constexpr (!EARLY) {
    if constexpr (I8) {
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          swv[i][g] = sw ? bias4(sw, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, N) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < FM; j++) sav[j] = sa ? sa[min(m0 + wm * WTM + j * 32 + lr, M - 1)] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        bv[i][g] = bias ? bias4(bias, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, N) : f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (HOIST_R) {
      if (R) {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
          for (int j = 0; j < FM; j++)
#pragma unroll
            for (int g = 0; g < 4; g++)
              rv[i][j][g] = res4(R, ldr, r_rows, m0 + wm * WTM + j * 32 + lr, n0 + wn * WTN + i * 32 + 8 * g + 4 * hk, M, N);
      }
    }
  }
  __syncthreads();
  // the activation and the residual's presence are compile-time in the loop (one straight run per case)
  if (owner) with_act(act, [&](auto ac) {
    constexpr int ACT = decltype(ac)::value;
    auto run = [&](auto hrc) {
      constexpr int HR = decltype(hrc)::value;
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++)
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const int r = wm * WTM + j * 32 + lr, c = wn * WTN + i * 32 + 8 * g + 4 * hk;
            u32x2 rg = {0u, 0u};
            if constexpr (HR == 1) {
              if constexpr (HOIST_R)
                rg = rv[i][j][g];
              else
                rg = res4(R, ldr, r_rows, m0 + r, n0 + c, M, N);
            }
            const f32x4 a4 = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
            if constexpr (I8) {
              if constexpr (ACT != 3)
                stage_val<ACT, SP>(smem, r, c, epi_val<ACT, true, HR>(a4, bv[i][g], rg, HR == 1, n0 + c, act_ncols,
                                                                       sav[j], swv[i][g]));
            } else {
              stage_val<ACT, SP>(smem, r, c, epi_val<ACT, false, HR>(a4, bv[i][g], rg, HR == 1, n0 + c, act_ncols));
            }
          }
    };
    if (R)
      run(IntC<1>{});
    else
      run(IntC<0>{});
  });
  __syncthreads();
  if (act == 3)
    store_staged<BM, BN / 2, SP, NT>(smem, C, ldc, m0, n0 / 2, M, N / 2, tid);
  else
    store_staged<BM, BN, SP, NT>(smem, C, ldc, m0, n0, M, N, tid);
}

template <int BM, int BN, int WGM, int WGN, int S>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, long lda, const uint16_t* __restrict__ W, long ldw,
    const float* __restrict__ bias, const uint16_t* __restrict__ R, long ldr, int r_rows,
    uint16_t* __restrict__ C, long ldc, int M, int N, int K, int Kw, int act, int act_ncols,
    int tiles_m, int tiles_n, int splits, int kt_per_split, float* __restrict__ ws, int* __restrict__ cnt,
    float* __restrict__ P, long ldp, long p_split) {
  gemm_body<BM, BN, WGM, WGN, S, false>(A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols,
                                        tiles_m, tiles_n, splits, kt_per_split, ws, cnt, P, ldp, p_split, nullptr,
                                        nullptr);
}

// The 8-wave form of a 2 x 2 tile: two wave groups, each on half of every k-step (KS = 2)
template <int BM, int BN, int S>
__global__ __launch_bounds__(512) void gemm_bf16_kh2_kernel(
    const uint16_t* __restrict__ A, long lda, const uint16_t* __restrict__ W, long ldw,
    const float* __restrict__ bias, const uint16_t* __restrict__ R, long ldr, int r_rows,
    uint16_t* __restrict__ C, long ldc, int M, int N, int K, int Kw, int act, int act_ncols,
    int tiles_m, int tiles_n, int splits, int kt_per_split, float* __restrict__ ws, int* __restrict__ cnt,
    float* __restrict__ P, long ldp, long p_split) {
  gemm_body<BM, BN, 2, 2, S, false, 2>(A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols,
                                       tiles_m, tiles_n, splits, kt_per_split, ws, cnt, P, ldp, p_split, nullptr,
                                       nullptr);
}

// The residual + LayerNorm (RLN 1) or RMSNorm (RLN 2) form (RlnArgs): one k range per tile (no split-K), 4-wave
// 2 x 2 tiles
template <int BM, int BN, int S, int RLN = 1>
__global__ __launch_bounds__(256) void gemm_rln_kernel(const uint16_t* __restrict__ A, long lda,
                                                       const uint16_t* __restrict__ W, long ldw,
                                                       const float* __restrict__ bias, const uint16_t* __restrict__ R,
                                                       long ldr, int M, int N, int K, int Kw, int tiles_m, int tiles_n,
                                                       RlnArgs rl) {
  gemm_body<BM, BN, 2, 2, S, false, 1, RLN>(A, lda, W, ldw, bias, R, ldr, 0, nullptr, 0, M, N, K, Kw, 0, 0, tiles_m,
                                             tiles_n, 1, Kw / BK, nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr, rl);
}

// W8A8: C = epi(((float)(Aq Wq^T) * sa[m]) * sw[n] + bias[n]) (K, Kw, lda, ldw in 16-bit units); P (raw int32
// accumulators) when given
template <int BM, int BN, int WGM, int WGN, int S>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_i8_kernel(
    const uint16_t* __restrict__ A, long lda, const uint16_t* __restrict__ W, long ldw, const float* __restrict__ sa,
    const float* __restrict__ sw, const float* __restrict__ bias, const uint16_t* __restrict__ R, long ldr,
    int r_rows, uint16_t* __restrict__ C, long ldc, int M, int N, int K, int Kw, int act, int act_ncols, int tiles_m,
    int tiles_n, float* __restrict__ P, long ldp, int splits, int kt_per_split, long p_split) {
  gemm_body<BM, BN, WGM, WGN, S, true>(A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols,
                                       tiles_m, tiles_n, splits, kt_per_split, nullptr, nullptr, P, ldp, p_split, sa,
                                       sw);
}

// Wave-split-K kernel (see the header): 4 waves share the LDS ring of a BM x BN tile; wave w multiplies the k
// columns [16 w, 16 w + 16) of every 64-wide k-step into its own copy of the whole tile.
template <int BM, int BN, int S, int OCC>
__global__ __launch_bounds__(256, OCC) void gemm_ks_kernel(
    const uint16_t* __restrict__ A, long lda, const uint16_t* __restrict__ W, long ldw,
    const float* __restrict__ bias, const uint16_t* __restrict__ R, long ldr, int r_rows,
    uint16_t* __restrict__ C, long ldc, int M, int N, int K, int Kw, int act, int act_ncols, int tiles_m, int tiles_n,
    int splits, int kt_per_split, float* __restrict__ P, long ldp, long p_split) {
  static_assert(S >= 2, "at least a double buffer");
  constexpr int FM = BM / 32, FN = BN / 32;
  constexpr int QA = BM / 32, QW = BN / 32;  // DMA instructions per wave per stage
  constexpr int LPS = QA + QW;
  constexpr int STAGE = (BM + BN) * BK;      // elements per ring stage
  constexpr int G = FM * FN * 4;             // 4-column output groups per lane
  constexpr int RING_B = S * STAGE * 2, RED_B = 2 * G * 64 * 16;
  // the k loop's ring, reused after the loop for the two partial tiles of the cross-wave sum
  __shared__ __attribute__((aligned(1024))) uint8_t smem_b[RING_B > RED_B ? RING_B : RED_B];
  uint16_t* smem = reinterpret_cast<uint16_t*>(smem_b);
  f32x4* red = reinterpret_cast<f32x4*>(smem_b);

  int tile_m, tile_n, split;
  tile_of(blockIdx.x, tiles_m, tiles_n, splits, tile_m, tile_n, split);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int kt0 = split * kt_per_split;
  const int nk = min(Kw / BK, kt0 + kt_per_split) - kt0;  // k-steps of this split
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, hk = lane >> 5;
  const uint32_t sbase = lds_off(smem);

  const int drow = lane >> 3, dch = (lane & 7) ^ ((lane >> 4) | ((wave & 1) << 2));
  const uint16_t* a_src[QA];
  const uint16_t* w_src[QW];
#pragma unroll
  for (int q = 0; q < QA; q++) a_src[q] = A + (long)min(m0 + 8 * (q * 4 + wave) + drow, M - 1) * lda;
#pragma unroll
  for (int q = 0; q < QW; q++) w_src[q] = W + (long)min(n0 + 8 * (q * 4 + wave) + drow, N - 1) * ldw;
  auto issue = [&](int kt, int s) {
    const int kk = kt * BK + dch * 8;
    const int ka = kk < K ? kk : 0;
    const uint32_t st = sbase + (uint32_t)(s * STAGE * 2);
#pragma unroll
    for (int q = 0; q < QA; q++) dma16(a_src[q] + ka, __builtin_amdgcn_readfirstlane(st + (q * 4 + wave) * 1024));
#pragma unroll
    for (int q = 0; q < QW; q++)
      dma16(w_src[q] + kk, __builtin_amdgcn_readfirstlane(st + BM * 128 + (q * 4 + wave) * 1024));
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // Software pipeline, as in gemm_bf16_kernel: this wave's fragments of k-step it + 1 are read (into the other
  // register buffer) while the MFMAs of k-step it run, so the LDS latency, the barrier and the slot refill sit under
  // the matrix work. The prologue fills all S slots; the reads after the last k-step fetch a stale slot that is never
  // used. The loop runs k-steps in pairs so both register buffers have compile-time indices; when nk is odd the
  // second step of the last pair multiplies zeroed fragments (adds exact zeros) instead of branching around the
  // MFMAs (one copy of the MFMAs keeps one set of accumulator registers).
  const int c = 2 * wave + hk;  // this lane's 16-byte chunk of each 128-byte LDS row
  bf16x8 af[2][FM], wf[2][FN];
  auto read_frags = [&](int buf, const uint16_t* As) {
    const uint16_t* Ws = As + BM * BK;
#pragma unroll
    for (int j = 0; j < FM; j++) {
      const int r = j * 32 + lr;
      af[buf][j] = as_bf16x8(*reinterpret_cast<const u32x4*>(&As[r * BK + ((c ^ ((r >> 1) & 7)) << 3)]));
    }
#pragma unroll
    for (int i = 0; i < FN; i++) {
      const int r = i * 32 + lr;
      wf[buf][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&Ws[r * BK + ((c ^ ((r >> 1) & 7)) << 3)]));
    }
  };
  auto step = [&](auto cur_c, int it) {
    constexpr int CUR = decltype(cur_c)::value;
    __builtin_amdgcn_sched_barrier(0);
    // stage it + 1 has landed once at most (stages issued after it) x LPS loads are still in flight; the barrier ends
    // every wave's reads of slot it % S, which is refilled with stage it + S
    wait_stages<LPS, S - 2>(nk - 2 - it);
    __syncthreads();
    if (it + S < nk) issue(kt0 + it + S, it % S);
    if (it >= nk) {  // the padding step of an odd nk: zero operands
#pragma unroll
      for (int j = 0; j < FM; j++) af[CUR][j] = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
#pragma unroll
      for (int i = 0; i < FN; i++) wf[CUR][i] = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
    }
    read_frags(CUR ^ 1, smem + ((it + 1) % S) * STAGE);
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++) acc[i][j] = mfma32(wf[CUR][i], af[CUR][j], acc[i][j]);
    interleave_reads_mfma<FM + FN, FM * FN>();
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int s = 0; s < S; s++)
    if (s < nk) issue(kt0 + s, s);
  wait_stages<LPS, S - 1>(nk - 1);  // stage 0 has landed
  __syncthreads();
  read_frags(0, smem);
  for (int it = 0; it < nk; it += 2) {
    step(IntC<0>{}, it);
    step(IntC<1>{}, it + 1);
  }

  // ---- cross-wave sum in a fixed order, ((w0 + w2) + (w1 + w3)): waves 2-3 hand their tiles to waves 0-1 through
  // LDS, waves 0-1 write the two sums back, and every wave finishes a quarter of the groups (epilogue + store)
  auto put = [&](int slot) {
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          red[(slot * G + (i * FM + j) * 4 + g) * 64 + lane] = v;
        }
  };
  __syncthreads();  // every wave is done with the ring
  if (wave >= 2) put(wave - 2);
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const f32x4 v = red[(wave * G + (i * FM + j) * 4 + g) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; e++) acc[i][j][4 * g + e] += v[e];
        }
  }
  __syncthreads();
  if (wave < 2) put(wave);
  __syncthreads();
  // this wave's groups q = wave + 4 t: sums, then (fused epilogue) every bias / residual load before the first store
  constexpr int GW = G / 4;
  static_assert(G % 4 == 0, "groups split evenly over the waves");
  f32x4 vs[GW];
#pragma unroll
  for (int t = 0; t < GW; t++) {
    const int q = wave + 4 * t;
    vs[t] = red[q * 64 + lane] + red[(G + q) * 64 + lane];
  }
  auto row_of = [&](int t) { return m0 + ((wave + 4 * t) / 4) % FM * 32 + lr; };
  auto col_of = [&](int t) {
    const int q = wave + 4 * t;
    return n0 + q / (FM * 4) * 32 + 8 * (q % 4) + 4 * hk;
  };
  __syncthreads();  // every wave has its sums: the LDS becomes the staging tile
  if (P) {
    // raw fp32 partial sums, staged like the bf16 results
    constexpr int SPF = BN + 4;
    static_assert(BM * SPF * 4 <= sizeof(smem_b), "fp32 staging tile fits");
    float* stf = reinterpret_cast<float*>(smem_b);
#pragma unroll
    for (int t = 0; t < GW; t++)
      *reinterpret_cast<f32x4*>(stf + (row_of(t) - m0) * SPF + (col_of(t) - n0)) = vs[t];
    __syncthreads();
    store_staged<BM, BN, SPF>(stf, P + split * p_split, ldp, m0, n0, M, N, tid);
    return;
  }
  // every bias / residual load issued before the first use (one latency for the lot)
  f32x4 bv[GW];
  u32x2 rv[GW];
#pragma unroll
  for (int t = 0; t < GW; t++) {
    bv[t] = bias ? bias4(bias, col_of(t), N) : f32x4{0.f, 0.f, 0.f, 0.f};
    rv[t] = R ? res4(R, ldr, r_rows, row_of(t), col_of(t), M, N) : u32x2{0u, 0u};
  }
  constexpr int SP = BN + 8;
  static_assert(BM * SP * 2 <= sizeof(smem_b), "staging tile fits");
  with_act(act, [&](auto ac) {
    constexpr int ACT = decltype(ac)::value;
#pragma unroll
    for (int t = 0; t < GW; t++) {
      const int n = col_of(t);
      stage_val<ACT, SP>(smem, row_of(t) - m0, n - n0, epi_val<ACT>(vs[t], bv[t], rv[t], R != nullptr, n, act_ncols));
    }
  });
  __syncthreads();
  if (act == 3)
    store_staged<BM, BN / 2, SP>(smem, C, ldc, m0, n0 / 2, M, N / 2, tid);
  else
    store_staged<BM, BN, SP>(smem, C, ldc, m0, n0, M, N, tid);
}

struct Cfg { int bm, bn, stages, per_cu, kind, waves, kh = 1; };
// kind 0: LDS-shared tile split over the waves; kind 1: wave-split K (each wave the whole tile, a quarter of K).
// Both stage operands through a `stages`-deep LDS ring.
// per_cu: workgroups that fit one CU at once (LDS- or register-limited)
constexpr Cfg kCfgs[] = {{128, 128, 4, 1, 0, 4}, {64, 128, 4, 1, 0, 4}, {128, 64, 4, 1, 0, 4}, {64, 64, 4, 2, 0, 4},
                         {256, 128, 3, 1, 0, 4}, {128, 256, 3, 1, 0, 4}, {64, 64, 3, 3, 0, 4}, {128, 128, 2, 2, 0, 4},
                         {64, 64, 4, 2, 1, 4},   {64, 128, 4, 1, 1, 4},  {128, 64, 4, 1, 1, 4}, {64, 64, 3, 3, 1, 4},
                         {64, 96, 2, 3, 1, 4},   {64, 64, 6, 1, 1, 4},   {96, 64, 2, 3, 1, 4},
                         // 8-wave tiles for large grids: 2 waves per SIMD hide each other's LDS reads and barriers
                         {256, 256, 2, 1, 0, 8}, {256, 128, 3, 1, 0, 8}, {128, 256, 3, 1, 0, 8},
                         // 4 waves of 128 x 128: 8 LDS reads per 16 MFMAs (LDS traffic at 3/4 of the MFMA time)
                         {256, 256, 2, 1, 0, 4},
                         // 8-wave forms of the 2 x 2 tiles, two k groups (kh = 2): batch-1 grids, one workgroup per
                         // CU, whose k loop waits on LDS reads at the 4-wave rate
                         {128, 128, 4, 1, 0, 8, 2}, {64, 128, 4, 1, 0, 8, 2}, {128, 64, 4, 1, 0, 8, 2},
                         {64, 64, 4, 2, 0, 8, 2},
                         // one wave row x 4 wave columns, 3 x 1 MFMA blocks per wave: 96-row tiles for M = 729
                         // (8 row tiles, the same 768 padded rows as 128 and a third more workgroups)
                         {96, 128, 4, 1, 0, 4},
                         // large grids whose N is a multiple of 192 (1152, 3456): 192 x 192 over two k groups with a
                         // 3-stage ring (two stages in flight), and 256 x 192 on 4 x 2 waves
                         {192, 192, 3, 1, 0, 8, 2}, {256, 192, 2, 1, 0, 8},
                         // 730-row prompt-prefix GEMMs: 4 row tiles of 192 x 64 column tiles of 128 = 256 workgroups
                         // for N = 8192; two k groups of 2 x 2 waves, 4-stage ring
                         {192, 128, 4, 1, 0, 8, 2}, {128, 192, 4, 1, 0, 8, 2}};
constexpr int kNCfg = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int BM, int BN, int WGM, int WGN, int S>
hipError_t launch(hipStream_t st, int splits, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                  const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N,
                  int K, int Kw, int act, int act_ncols, float* ws, int* cnt, float* P = nullptr, long ldp = 0,
                  long p_split = 0) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int nk = Kw / BK;
  const int kps = (nk + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WGM, WGN, S>), dim3(tm * tn * splits), dim3(64 * WGM * WGN), 0, st, A, lda, W,
                     ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, tm, tn, splits, kps, ws, cnt, P,
                     ldp, p_split);
  return hipGetLastError();
}

template <int BM, int BN, int S>
hipError_t launch_kh2(hipStream_t st, int splits, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                      const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N,
                      int K, int Kw, int act, int act_ncols, float* P = nullptr, long ldp = 0, long p_split = 0) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int nk = Kw / BK;
  const int kps = (nk + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_bf16_kh2_kernel<BM, BN, S>), dim3(tm * tn * splits), dim3(512), 0, st, A, lda, W, ldw, bias,
                     R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, tm, tn, splits, kps, nullptr, nullptr, P,
                     ldp, p_split);
  return hipGetLastError();
}

template <int BM, int BN, int S, int OCC>
hipError_t launch_ks(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
                     const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int K, int Kw,
                     int act, int act_ncols, int splits = 1, float* P = nullptr, long ldp = 0, long p_split = 0) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int nk = Kw / BK, kps = (nk + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_ks_kernel<BM, BN, S, OCC>), dim3(tm * tn * splits), dim3(256), 0, st, A, lda, W, ldw, bias, R, ldr,
                     r_rows, C, ldc, M, N, K, Kw, act, act_ncols, tm, tn, splits, kps, P, ldp, p_split);
  return hipGetLastError();
}

// configs with a partial-sum mode (mx_gemm_bf16_partial) and in-kernel split-K: every wave-split config, and the
// 4-wave kind-0 tiles whose fp32 staging tile fits the LDS (the kernel's PSUM)
bool psum_ok(int cfg) {
  const Cfg& c = kCfgs[cfg];
  return c.kind == 1 || (c.waves / c.kh == 4 && c.bm * c.bn <= 128 * 256);
}

template <int BM, int BN, int WGM, int WGN, int S>
hipError_t launch_i8(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* sa,
                     const float* sw, const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C,
                     long ldc, int M, int N, int K, int Kw, int act, float* P, long ldp, int splits = 1,
                     long p_split = 0) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int nk = Kw / BK, kps = (nk + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WGM, WGN, S>), dim3(tm * tn * splits), dim3(64 * WGM * WGN), 0, st, A, lda,
                     W, ldw, sa, sw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, 0, tm, tn, P, ldp, splits, kps,
                     p_split);
  return hipGetLastError();
}

long tiles_of(int cfg, int M, int N) {
  return (long)((M + kCfgs[cfg].bm - 1) / kCfgs[cfg].bm) * ((N + kCfgs[cfg].bn - 1) / kCfgs[cfg].bn);
}

// ---- split-K reduction + epilogue: C = epi(sum_s P[s] + bias) with the fused kernel's epilogue (epi_val), so one
// split of raw partials reduced here equals the fused GEMM bit for bit. One thread per 4 output columns; the splits
// are added in order (deterministic).
template <int ACT>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ P, int ns, long p_split, long ldp,
                                                          const float* __restrict__ bias, const uint16_t* __restrict__ R,
                                                          long ldr, int r_rows, uint16_t* __restrict__ C, long ldc,
                                                          int M, int N, int act_ncols) {
  const int n4 = N >> 2;
  const long total = (long)M * n4;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    const int m = (int)(i / n4), n = (int)(i % n4) * 4;
    const float* pp = P + (long)m * ldp + n;
    f32x4 acc = *reinterpret_cast<const f32x4*>(pp);
    for (int sp = 1; sp < ns; sp++) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(pp + sp * p_split);
#pragma unroll
      for (int e = 0; e < 4; e++) acc[e] = acc[e] + t[e];
    }
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
#pragma unroll
      for (int e = 0; e < 4; e++) bv[e] = bias[n + e];
    }
    u32x2 rv = {0u, 0u};
    if (R) rv = *reinterpret_cast<const u32x2*>(R + (long)(r_rows > 0 ? m % r_rows : m) * ldr + n);
    const u32x2 o = epi_val<ACT>(acc, bv, rv, R != nullptr, n, act_ncols);
    if constexpr (ACT == 3)
      *reinterpret_cast<uint32_t*>(C + (long)m * ldc + (n >> 1)) = o.x;
    else
      *reinterpret_cast<u32x2*>(C + (long)m * ldc + n) = o;
  }
}

// The W8A8 form: int32 partials summed exactly, then epi_val's int8 epilogue (it takes the int32 sum as the bit
// pattern of an fp32 register, as the tile kernel hands it its accumulator).
template <int ACT>
__global__ __launch_bounds__(256) void gemm_reduce_i8_kernel(const int32_t* __restrict__ P, int ns, long p_split,
                                                             long ldp, const float* __restrict__ sa,
                                                             const float* __restrict__ sw,
                                                             const float* __restrict__ bias,
                                                             const uint16_t* __restrict__ R, long ldr, int r_rows,
                                                             uint16_t* __restrict__ C, long ldc, int M, int N) {
  const int n4 = N >> 2;
  const long total = (long)M * n4;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    const int m = (int)(i / n4), n = (int)(i % n4) * 4;
    const int32_t* pp = P + (long)m * ldp + n;
    int32_t acc[4] = {pp[0], pp[1], pp[2], pp[3]};
    for (int sp = 1; sp < ns; sp++) {
      const u32x4 t = *reinterpret_cast<const u32x4*>(pp + sp * p_split);
#pragma unroll
      for (int e = 0; e < 4; e++) acc[e] += (int32_t)t[e];
    }
    f32x4 s, bv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; e++) s[e] = __int_as_float(acc[e]);
    if (bias) {
#pragma unroll
      for (int e = 0; e < 4; e++) bv[e] = bias[n + e];
    }
    const f32x4 sw4 = *reinterpret_cast<const f32x4*>(sw + n);
    u32x2 rv = {0u, 0u};
    if (R) rv = *reinterpret_cast<const u32x2*>(R + (long)(r_rows > 0 ? m % r_rows : m) * ldr + n);
    *reinterpret_cast<u32x2*>(C + (long)m * ldc + n) = epi_val<ACT, true>(s, bv, rv, R != nullptr, n, 0, sa[m], sw4);
  }
}

}  // namespace

extern "C" int mx_gemm_ncfg(void) { return kNCfg; }

extern "C" int mx_gemm_cfg_tile(int cfg, int* bm, int* bn) {
  if (cfg < 0 || cfg >= kNCfg) return MX_EBADCFG;
  *bm = kCfgs[cfg].bm;
  *bn = kCfgs[cfg].bn;
  return MX_OK;
}

extern "C" int mx_gemm_cfg_kind(int cfg) {
  if (cfg < 0 || cfg >= kNCfg) return MX_EBADCFG;
  return kCfgs[cfg].kind;
}

// Workspace a (cfg, splits) call needs: fp32 partial tiles and one counter per output tile.
extern "C" long mx_gemm_ws_elems(int cfg, int splits, int M, int N) {
  if (cfg < 0 || cfg >= kNCfg || splits <= 1 || kCfgs[cfg].kind) return 0;
  return tiles_of(cfg, M, N) * splits * kCfgs[cfg].bm * kCfgs[cfg].bn;
}
extern "C" long mx_gemm_ws_counters(int cfg, int splits, int M, int N) {
  if (cfg < 0 || cfg >= kNCfg || splits <= 1 || kCfgs[cfg].kind) return 0;
  return tiles_of(cfg, M, N);
}

// Default (cfg, splits) when the caller passes cfg < 0: minimise estimated time = rounds of workgroups over the
// 256 CUs x per-tile time, with per-tile time ~ BM*BN*(k-steps)/efficiency. Returns cfg * 16 + splits.
extern "C" int mx_gemm_pick(int M, int N, int Kw) {
  static const float eff[] = {1.0f, 0.78f, 0.78f, 0.6f, 1.1f, 1.1f, 0.6f, 0.9f, 1.0f, 1.0f, 1.0f, 1.0f,
                              1.0f, 1.0f, 1.0f, 1.3f, 1.1f, 1.1f, 1.4f, 1.1f, 0.9f, 0.9f, 0.7f, 0.9f,
                              1.2f, 1.2f, 1.1f, 1.1f};
  static_assert(sizeof eff / sizeof eff[0] == kNCfg, "one efficiency per tile config");
  const int nk = Kw / BK;
  int best = 0, bsplit = 1;
  float bt = 1e30f;
  for (int c = 0; c < kNCfg; c++) {
    for (int sp = 1; sp <= 8; sp *= 2) {
      if (sp > 1 && (kCfgs[c].kind || kCfgs[c].kh != 1 || !psum_ok(c) || nk / sp < 4 || (sp - 1) * ((nk + sp - 1) / sp) >= nk))
        break;
      const long tiles = tiles_of(c, M, N) * sp;
      const long slots = 256L * kCfgs[c].per_cu;
      const long rounds = (tiles + slots - 1) / slots;
      const float tk = (float)((nk + sp - 1) / sp);
      float t = (float)rounds * kCfgs[c].bm * kCfgs[c].bn * (tk + 2.0f) / eff[c];
      if (sp > 1) t *= 4.0f;  // partial-tile traffic and the cross-XCD release fence of the reduction
      if (t < bt) { bt = t; best = c; bsplit = sp; }
    }
  }
  return best * 16 + bsplit;
}

// Validate a GEMM call without launching (0 or a negative status).
extern "C" int mx_gemm_check(int cfg, int splits, const void* A, long lda, const void* W, long ldw, const void* bias,
                             const void* R, long ldr, const void* C, long ldc, int M, int N, int K, int Kw, int act,
                             const void* ws, long ws_elems, const void* cnt, long n_cnt) {
  if (!A || !W || !C) return MX_ENULL;
  if (cfg >= kNCfg) return MX_EBADCFG;
  if (act < 0 || act > 3) return MX_EBADCFG;
  if (M < 1 || N < 1 || K < 8) return MX_ESHAPE;
  if (K % 8 || Kw % BK || Kw < K || lda % 8 || ldw % 8 || lda < K || ldw < Kw) return MX_ESHAPE;
  if (N % 4 || ldc % 2 || ldc < (act == 3 ? N / 2 : N) || (act != 3 && ldc % 4)) return MX_ESHAPE;
  if (act == 3 && R) return MX_EBADCFG;
  if (((uintptr_t)A | (uintptr_t)W) & 15) return MX_ELAYOUT;
  if ((uintptr_t)C & 7) return MX_ELAYOUT;
  if (bias && ((uintptr_t)bias & 15)) return MX_ELAYOUT;
  if (R && (((uintptr_t)R & 7) || ldr % 4 || ldr < N)) return MX_ELAYOUT;
  if (cfg >= 0 && splits > 1) {
    if (kCfgs[cfg].kind || kCfgs[cfg].kh != 1 || !psum_ok(cfg)) return MX_ESPLIT;  // 4-wave kind-0 tiles up to 128 x 256
    const int nk = Kw / BK, kps = (nk + splits - 1) / splits;
    if (splits > nk || (splits - 1) * kps >= nk) return MX_ESPLIT;  // every split must own >= 1 k-step
    if (!ws || !cnt) return MX_ENULL;
    if (ws_elems < mx_gemm_ws_elems(cfg, splits, M, N) || n_cnt < mx_gemm_ws_counters(cfg, splits, M, N))
      return MX_ESPLIT;
  }
  return MX_OK;
}

// C = epi(A W^T + bias). cfg < 0: the library's pick (only split-free picks unless a workspace is given).
// ws / cnt: split-K workspace (fp32 elements) and per-tile counters (must be zero before first use; the kernel
// leaves them zero). R row for output row m is (r_rows > 0 ? m % r_rows : m).
// act: 0 none, 1 GELU-tanh, 2 GELU-erf, 3 gated GELU-tanh on interleaved (gate, up) weight-row pairs (output width
// N / 2: column j = bf16(bf16(gelu(gate_j)) * up_j) with gate_j / up_j = linear rows 2 j / 2 j + 1). act 1-2 apply
// to output columns < act_ncols only when act_ncols > 0 (e.g. GELU on the y half of a fused [y | x] projection).
extern "C" int mx_gemm_bf16(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda, const uint16_t* W,
                            long ldw, const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C,
                            long ldc, int M, int N, int K, int Kw, int act, int act_ncols, float* ws, long ws_elems,
                            int* cnt, long n_cnt) {
  if (r_rows < 0) return MX_ESHAPE;
  if (cfg < 0) {
    const int p = mx_gemm_pick(M, N, Kw);
    cfg = p / 16;
    splits = p % 16;
    if (splits > 1 && (ws_elems < mx_gemm_ws_elems(cfg, splits, M, N) || n_cnt < mx_gemm_ws_counters(cfg, splits, M, N)))
      splits = 1;
  }
  if (splits < 1) splits = 1;
  const int rc = mx_gemm_check(cfg, splits, A, lda, W, ldw, bias, R, ldr, C, ldc, M, N, K, Kw, act, ws, ws_elems, cnt, n_cnt);
  if (rc) return rc;
  hipError_t e;
#define L_(BM, BN, S) launch<BM, BN, 2, 2, S>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt)
  switch (cfg) {
    case 0: e = L_(128, 128, 4); break;
    case 1: e = L_(64, 128, 4); break;
    case 2: e = L_(128, 64, 4); break;
    case 3: e = L_(64, 64, 4); break;
    case 4: e = L_(256, 128, 3); break;
    case 5: e = L_(128, 256, 3); break;
    case 6: e = L_(64, 64, 3); break;
    case 7: e = L_(128, 128, 2); break;
    case 23: e = launch<96, 128, 1, 4, 4>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt); break;
    case 15: e = launch<256, 256, 2, 4, 2>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt); break;
    case 16: e = launch<256, 128, 4, 2, 3>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt); break;
    case 17: e = launch<128, 256, 2, 4, 3>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt); break;
    case 18: e = L_(256, 256, 2); break;
    case 25: e = launch<256, 192, 4, 2, 2>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws, cnt); break;
#define H_(BM, BN, S) launch_kh2<BM, BN, S>(st, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols)
    case 19: e = H_(128, 128, 4); break;
    case 20: e = H_(64, 128, 4); break;
    case 21: e = H_(128, 64, 4); break;
    case 22: e = H_(64, 64, 4); break;
    case 24: e = H_(192, 192, 3); break;
    case 26: e = H_(192, 128, 4); break;
    case 27: e = H_(128, 192, 4); break;
#define W_(BM, BN, S, OCC) launch_ks<BM, BN, S, OCC>(st, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols)
    case 8: e = W_(64, 64, 4, 2); break;
    case 9: e = W_(64, 128, 4, 1); break;
    case 10: e = W_(128, 64, 4, 1); break;
    case 11: e = W_(64, 64, 3, 3); break;
    case 12: e = W_(64, 96, 2, 3); break;
    case 13: e = W_(64, 64, 6, 1); break;
    case 14: e = W_(96, 64, 2, 3); break;
    default: return MX_EBADCFG;
  }
#undef L_
#undef W_
#undef H_
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// ---------------------------------------------------------------------------------------------- allocation-free form
// mx_gemm_bf16 for callers that cannot allocate (code under HIP-graph capture, tight serving loops, harnesses that
// forbid hipMalloc): the split-K workspace is a fixed file-scope device array instead of a caller buffer. Each GPU
// holds its own copy for the life of the process; its address is looked up once per device with the device current
// (host code never passes the array's name itself to a kernel). Calls on one GPU share it: two such calls that
// overlap on that GPU (on different streams) race.
constexpr long kScratchWs = 4L << 20;   // fp32 partial-tile elements (16 MiB)
constexpr long kScratchCnt = 1L << 16;  // per-tile arrival counters
static __device__ __align__(256) float scratch[kScratchWs + kScratchCnt];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

float* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

__global__ void zero_ints_kernel(int* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0;
}
}  // namespace

extern "C" long mx_gemm_noalloc_max_ws(void) { return kScratchWs; }

extern "C" int mx_gemm_bf16_noalloc(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda, const uint16_t* W,
                                    long ldw, const float* bias, const uint16_t* R, long ldr, int r_rows, uint16_t* C,
                                    long ldc, int M, int N, int K, int Kw, int act, int act_ncols) {
  if (cfg < 0) {
    const int p = mx_gemm_pick(M, N, Kw);
    cfg = p / 16;
    splits = p % 16;
    if (splits > 1 && (mx_gemm_ws_elems(cfg, splits, M, N) > kScratchWs ||
                       mx_gemm_ws_counters(cfg, splits, M, N) > kScratchCnt))
      splits = 1;
  }
  if (splits < 1) splits = 1;
  float* ws = nullptr;
  int* cnt = nullptr;
  long ncnt = 0;
  if (splits > 1) {
    if (cfg >= kNCfg) return MX_EBADCFG;
    const long need = mx_gemm_ws_elems(cfg, splits, M, N);
    ncnt = mx_gemm_ws_counters(cfg, splits, M, N);
    if (need > kScratchWs || ncnt > kScratchCnt) return MX_ESPLIT;  // beyond the fixed workspace
    ws = scratch_ptr();
    if (!ws) return MX_ELAUNCH;
    cnt = reinterpret_cast<int*>(ws + kScratchWs);
    const int rc = mx_gemm_check(cfg, splits, A, lda, W, ldw, bias, R, ldr, C, ldc, M, N, K, Kw, act, ws, kScratchWs,
                                 cnt, kScratchCnt);
    if (rc) return rc;
    // the counters must start at zero: a kernel clears them (no memset node, so the call stays graph-capturable)
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)((ncnt + 255) / 256)), dim3(256), 0, st, cnt, ncnt);
    if (hipGetLastError() != hipSuccess) return MX_ELAUNCH;
  }
  return mx_gemm_bf16(st, cfg, splits, A, lda, W, ldw, bias, R, ldr, r_rows, C, ldc, M, N, K, Kw, act, act_ncols, ws,
                      splits > 1 ? kScratchWs : 0, cnt, splits > 1 ? kScratchCnt : 0);
}

// C = epi(sum over s < nsplit of P[s] + bias): the epilogue of mx_gemm_bf16 (act 0 / 1 / 2 on columns < act_ncols when
// act_ncols > 0, 3 = gated GELU on interleaved (gate, up) column pairs with output width N / 2; then + R) on raw
// partials from mx_gemm_bf16_partial, splits added in order. Partial GEMM + this reduction is the fence-free
// split-K: no counters, no cross-workgroup visibility inside a launch (stream order is the only synchronisation).
// No counterpart in the reference; it stands for the small-M split-K path of i8gemm_small_launch
// (moondream/gpu/hip/i8gemm.hip:555-592) on the bf16 side.
extern "C" int mx_gemm_reduce(hipStream_t st, const float* P, int nsplit, long p_split, long ldp, const float* bias,
                              const uint16_t* R, long ldr, int r_rows, uint16_t* C, long ldc, int M, int N, int act,
                              int act_ncols) {
  if (!P || !C) return MX_ENULL;
  if (nsplit < 1 || nsplit > 64 || M < 1 || N < 4 || N % 4 || ldp % 4 || ldp < N || act < 0 || act > 3 ||
      r_rows < 0 || (nsplit > 1 && p_split < (long)M * ldp) || p_split % 4)
    return MX_ESHAPE;
  if (act == 3 ? (ldc < N / 2 || ldc % 2) : (ldc < N || ldc % 4)) return MX_ESHAPE;
  if (R && (ldr < N || ldr % 4 || act == 3)) return MX_ESHAPE;
  if (((uintptr_t)P & 15) || ((uintptr_t)C & (act == 3 ? 3 : 7)) || ((uintptr_t)R & 7)) return MX_ELAYOUT;
  const long total = (long)M * (N / 4);
  const int blocks = (int)((total + 255) / 256 < 2048 ? (total + 255) / 256 : 2048);
#define RL_(A) hipLaunchKernelGGL((gemm_reduce_kernel<A>), dim3(blocks), dim3(256), 0, st, P, nsplit, p_split, ldp, bias, R, ldr, r_rows, C, ldc, M, N, act_ncols)
  switch (act) {
    case 0: RL_(0); break;
    case 1: RL_(1); break;
    case 2: RL_(2); break;
    default: RL_(3); break;
  }
#undef RL_
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// W8A8 split-K: raw int32 partials of S splits of the int8 GEMM (the same tile kernel in its raw mode, each split a
// contiguous range of k-steps). Integer sums are exact in any order, so partials + mx_gemm_i8_reduce equal
// mx_gemm_i8 bit for bit whatever the split count.
extern "C" int mx_gemm_i8_partial(hipStream_t st, int cfg, int splits, const int8_t* A, long lda, const int8_t* W,
                                  long ldw, int32_t* P, long ldp, long p_split, int M, int N, int K, int Kw) {
  if (!A || !W || !P) return MX_ENULL;
  if (cfg < 0 || cfg >= kNCfg || kCfgs[cfg].kind != 0 || !psum_ok(cfg)) return MX_EBADCFG;
  if (M < 1 || N < 1 || N % 4 || K < 16 || K % 16 || Kw % 128 || Kw < K) return MX_ESHAPE;
  if (lda % 16 || lda < K || ldw % 16 || ldw < Kw) return MX_ESHAPE;
  const int nk = Kw / 128;
  if (splits < 1 || splits > nk) return MX_ESPLIT;
  const int kps = (nk + splits - 1) / splits;
  if ((splits - 1) * kps >= nk) return MX_ESPLIT;  // every split owns >= 1 k-step
  if (ldp % 4 || ldp < N || ((uintptr_t)P & 15) || p_split % 4 || (splits > 1 && p_split < (long)M * ldp))
    return MX_ELAYOUT;
  if (((uintptr_t)A | (uintptr_t)W) & 15) return MX_ELAYOUT;
  const uint16_t* A16 = reinterpret_cast<const uint16_t*>(A);
  const uint16_t* W16 = reinterpret_cast<const uint16_t*>(W);
  float* Pf = reinterpret_cast<float*>(P);
  hipError_t e;
#define I_(BM, BN, WGM, WGN, S) launch_i8<BM, BN, WGM, WGN, S>(st, A16, lda / 2, W16, ldw / 2, nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr, 0, M, N, K / 2, Kw / 2, 0, Pf, ldp, splits, p_split)
  switch (cfg) {
    case 0: e = I_(128, 128, 2, 2, 4); break;
    case 1: e = I_(64, 128, 2, 2, 4); break;
    case 2: e = I_(128, 64, 2, 2, 4); break;
    case 3: e = I_(64, 64, 2, 2, 4); break;
    case 4: e = I_(256, 128, 2, 2, 3); break;
    case 5: e = I_(128, 256, 2, 2, 3); break;
    case 6: e = I_(64, 64, 2, 2, 3); break;
    case 7: e = I_(128, 128, 2, 2, 2); break;
    case 23: e = I_(96, 128, 1, 4, 4); break;
    default: return MX_EBADCFG;
  }
#undef I_
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// C = the W8A8 epilogue of mx_gemm_i8 (((float)acc * sa[m]) * sw[n] + bias[n], act 0 / 1 / 2 on that fp32 value, one
// bf16 rounding, then + R) on acc = the int32 sum of nsplit raw partials. sw 16-byte aligned.
extern "C" int mx_gemm_i8_reduce(hipStream_t st, const int32_t* P, int nsplit, long p_split, long ldp, const float* sa,
                                 const float* sw, const float* bias, const uint16_t* R, long ldr, int r_rows,
                                 uint16_t* C, long ldc, int M, int N, int act) {
  if (!P || !C || !sa || !sw) return MX_ENULL;
  if (nsplit < 1 || nsplit > 64 || M < 1 || N < 4 || N % 4 || ldp % 4 || ldp < N || act < 0 || act > 2 ||
      r_rows < 0 || (nsplit > 1 && p_split < (long)M * ldp) || p_split % 4 || ldc < N || ldc % 4)
    return MX_ESHAPE;
  if (R && (ldr < N || ldr % 4)) return MX_ESHAPE;
  if (((uintptr_t)P & 15) || ((uintptr_t)C & 7) || ((uintptr_t)R & 7) || ((uintptr_t)sw & 15)) return MX_ELAYOUT;
  const long total = (long)M * (N / 4);
  const int blocks = (int)((total + 255) / 256 < 2048 ? (total + 255) / 256 : 2048);
#define RL_(A) hipLaunchKernelGGL((gemm_reduce_i8_kernel<A>), dim3(blocks), dim3(256), 0, st, P, nsplit, p_split, ldp, sa, sw, bias, R, ldr, r_rows, C, ldc, M, N)
  switch (act) {
    case 0: RL_(0); break;
    case 1: RL_(1); break;
    default: RL_(2); break;
  }
#undef RL_
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Raw split-K partial sums of A W^T for wave-split configs (kind 1): P[s][m][n] (fp32, row stride ldp, split stride
// p_split) = sum over the k-steps of split s, s < splits. No bias, activation or residual: the consumer reduces the
// splits in order (e.g. mx_residual_layernorm). No counterpart in the reference, which has no split-K.
extern "C" int mx_gemm_bf16_partial(hipStream_t st, int cfg, int splits, const uint16_t* A, long lda,
                                    const uint16_t* W, long ldw, float* P, long ldp, long p_split, int M, int N, int K,
                                    int Kw) {
  if (cfg < 0 || cfg >= kNCfg || !psum_ok(cfg)) return MX_EBADCFG;
  if (!P) return MX_ENULL;
  int rc = mx_gemm_check(cfg, 1, A, lda, W, ldw, nullptr, nullptr, 0, P, ldp, M, N, K, Kw, 0, nullptr, 0, nullptr, 0);
  if (rc) return rc;
  const int nk = Kw / BK;
  if (splits < 1 || splits > nk) return MX_ESPLIT;
  const int kps = (nk + splits - 1) / splits;
  if ((splits - 1) * kps >= nk) return MX_ESPLIT;  // every split owns >= 1 k-step
  if (ldp % 4 || ldp < N || ((uintptr_t)P & 15) || p_split % 4 || (splits > 1 && p_split < (long)M * ldp))
    return MX_ELAYOUT;
  hipError_t e;
#define W_(BM, BN, S, OCC) launch_ks<BM, BN, S, OCC>(st, A, lda, W, ldw, nullptr, nullptr, 0, 0, nullptr, 0, M, N, K, Kw, 0, 0, splits, P, ldp, p_split)
#define L_(BM, BN, S) launch<BM, BN, 2, 2, S>(st, splits, A, lda, W, ldw, nullptr, nullptr, 0, 0, nullptr, 0, M, N, K, Kw, 0, 0, nullptr, nullptr, P, ldp, p_split)
  switch (cfg) {
    case 0: e = L_(128, 128, 4); break;
    case 1: e = L_(64, 128, 4); break;
    case 2: e = L_(128, 64, 4); break;
    case 3: e = L_(64, 64, 4); break;
    case 4: e = L_(256, 128, 3); break;
    case 5: e = L_(128, 256, 3); break;
    case 6: e = L_(64, 64, 3); break;
    case 7: e = L_(128, 128, 2); break;
    case 23: e = launch<96, 128, 1, 4, 4>(st, splits, A, lda, W, ldw, nullptr, nullptr, 0, 0, nullptr, 0, M, N, K, Kw, 0, 0, nullptr, nullptr, P, ldp, p_split); break;
#define H_(BM, BN, S) launch_kh2<BM, BN, S>(st, splits, A, lda, W, ldw, nullptr, nullptr, 0, 0, nullptr, 0, M, N, K, Kw, 0, 0, P, ldp, p_split)
    case 19: e = H_(128, 128, 4); break;
    case 20: e = H_(64, 128, 4); break;
    case 21: e = H_(128, 64, 4); break;
    case 22: e = H_(64, 64, 4); break;
    case 26: e = H_(192, 128, 4); break;
    case 27: e = H_(128, 192, 4); break;
#undef H_
    case 8: e = W_(64, 64, 4, 2); break;
    case 9: e = W_(64, 128, 4, 1); break;
    case 10: e = W_(128, 64, 4, 1); break;
    case 11: e = W_(64, 64, 3, 3); break;
    case 12: e = W_(64, 96, 2, 3); break;
    case 13: e = W_(64, 64, 6, 1); break;
    case 14: e = W_(96, 64, 2, 3); break;
    default: return MX_EBADCFG;
  }
#undef W_
#undef L_
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// W8A8 GEMM (the reference's HI8Lin path, moondream/gpu/hgemm.py:95-137 / i8gemm.hip:91-201 with bias, optional GELU
// and, beyond the reference, an optional fused residual): C = bf16(gelu?(((float)(A W^T) * sa[m]) * sw[n] + bias[n]))
// [+ R, rounded again]. A (M, K) and W (N, Kw) are int8 with row strides lda / ldw in bytes; W holds zeros in columns
// [K, Kw); sa (M) and sw (N) are the fp32 row / column scales. With P, the raw int32 accumulators go to P (row stride
// ldp elements) instead: no scales, bias, activation or C. cfg: a kind-0 tile config (mx_gemm_cfg_kind 0; P needs
// one with a partial-sum mode); act: 0 none, 1 GELU-tanh, 2 GELU-erf. No split-K.
extern "C" int mx_gemm_i8(hipStream_t st, int cfg, const int8_t* A, long lda, const int8_t* W, long ldw,
                          const float* sa, const float* sw, const float* bias, const uint16_t* R, long ldr, int r_rows,
                          uint16_t* C, long ldc, int M, int N, int K, int Kw, int act, int32_t* P, long ldp) {
  if (!A || !W) return MX_ENULL;
  if (!P && (!C || !sa || !sw)) return MX_ENULL;
  if (cfg < 0 || cfg >= kNCfg || kCfgs[cfg].kind != 0) return MX_EBADCFG;
  if (P && !psum_ok(cfg)) return MX_EBADCFG;
  if (act < 0 || act > 2) return MX_EBADCFG;
  if (M < 1 || N < 1 || N % 4 || K < 16 || K % 16 || Kw % 128 || Kw < K) return MX_ESHAPE;
  if (lda % 16 || lda < K || ldw % 16 || ldw < Kw || r_rows < 0) return MX_ESHAPE;
  if (((uintptr_t)A | (uintptr_t)W) & 15) return MX_ELAYOUT;
  if (P) {
    if (ldp % 4 || ldp < N || ((uintptr_t)P & 15)) return MX_ELAYOUT;
  } else {
    if (ldc % 4 || ldc < N || ((uintptr_t)C & 7)) return MX_ESHAPE;
    if (((uintptr_t)sw & 15) || (bias && ((uintptr_t)bias & 15))) return MX_ELAYOUT;
    if (R && (((uintptr_t)R & 7) || ldr % 4 || ldr < N)) return MX_ELAYOUT;
  }
  const uint16_t* A16 = reinterpret_cast<const uint16_t*>(A);
  const uint16_t* W16 = reinterpret_cast<const uint16_t*>(W);
  float* Pf = reinterpret_cast<float*>(P);
  hipError_t e;
#define I_(BM, BN, WGM, WGN, S) launch_i8<BM, BN, WGM, WGN, S>(st, A16, lda / 2, W16, ldw / 2, sa, sw, bias, R, ldr, r_rows, C, ldc, M, N, K / 2, Kw / 2, act, Pf, ldp)
  switch (cfg) {
    case 0: e = I_(128, 128, 2, 2, 4); break;
    case 1: e = I_(64, 128, 2, 2, 4); break;
    case 2: e = I_(128, 64, 2, 2, 4); break;
    case 3: e = I_(64, 64, 2, 2, 4); break;
    case 4: e = I_(256, 128, 2, 2, 3); break;
    case 5: e = I_(128, 256, 2, 2, 3); break;
    case 6: e = I_(64, 64, 2, 2, 3); break;
    case 7: e = I_(128, 128, 2, 2, 2); break;
    case 23: e = I_(96, 128, 1, 4, 4); break;
    case 15: e = I_(256, 256, 2, 4, 2); break;
    case 16: e = I_(256, 128, 4, 2, 3); break;
    case 17: e = I_(128, 256, 2, 4, 3); break;
    case 18: e = I_(256, 256, 2, 2, 2); break;
    default: return MX_EBADCFG;
  }
#undef I_
  return e == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Residual Linear + LayerNorm in one launch: X = bf16(bf16(A W^T + bias) + R) (the residual stream) and
// Y = LayerNorm(X) with gamma, beta, eps (the next normalisation). Replaces the Linear with the residual
// (md2fast.py:154, :157 lin_res) and the LayerNorm that reads its output (:155 ln2, the next block's ln1 at :153),
// i.e. mx_gemm_bf16_partial + mx_residual_layernorm with one split. The row statistics combine the tiles' sums and
// centred square sums (exact identity for the centred sum of squares; fp32 summation in another order than the
// row kernel). stats: stats_words >= mx_gemm_res_ln_stats_words(M, N) 64-bit words; sync: sync_words >=
// mx_gemm_res_ln_sync_words(M) 32-bit words, zeroed once by the caller, then owned by it: calls that share them
// must be ordered on one stream. sync[0] != 0 after a call means a wait timed out (results undefined; zero sync
// and stats before the next call). Needs N a multiple of 64 (at most 4096) and a grid of at most one workgroup per
// CU ((M / 64 rounded up) x (N / 64) <= the device's CU count), else MX_ESHAPE.
extern "C" long mx_gemm_res_ln_stats_words(int M, int N) { return (long)((M + 63) / 64) * (N / 64) * 64 * 2; }
extern "C" long mx_gemm_res_ln_sync_words(int M) { return 1 + (long)((M + 63) / 64); }

namespace {
template <int RLN>
int launch_rln(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw, const float* bias,
               const uint16_t* R, long ldr, uint16_t* X, long ldx, const uint16_t* gamma, const uint16_t* beta,
               uint16_t* Y, long ldy, int M, int N, int K, int Kw, float eps, uint64_t* stats, long stats_words,
               uint32_t* sync, long sync_words) {
  if (!R || !X || !gamma || (RLN == 1 && !beta) || !Y || !stats || !sync) return MX_ENULL;
  int rc = mx_gemm_check(3, 1, A, lda, W, ldw, bias, R, ldr, X, ldx, M, N, K, Kw, 0, nullptr, 0, nullptr, 0);
  if (rc) return rc;
  if (N % 64 || N / 64 > kRlnMaxTiles) return MX_ESHAPE;
  if (ldy % 4 || ldy < N || ((uintptr_t)Y & 7) || (((uintptr_t)gamma | (uintptr_t)beta) & 7)) return MX_ELAYOUT;
  if (stats_words < mx_gemm_res_ln_stats_words(M, N) || sync_words < mx_gemm_res_ln_sync_words(M)) return MX_ESHAPE;
  if ((uintptr_t)stats & 15) return MX_ELAYOUT;
  const int tm = (M + 63) / 64, tn = N / 64;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return MX_ELAUNCH;
  if ((long)tm * tn > cus) return MX_ESHAPE;  // every tile of a row block resident at once
  const RlnArgs rl{gamma, beta, X, ldx, Y, ldy, eps, stats, sync};
  hipLaunchKernelGGL((gemm_rln_kernel<64, 64, 4, RLN>), dim3(tm * tn), dim3(256), 0, st, A, lda, W, ldw, bias, R, ldr,
                     M, N, K, Kw, tm, tn, rl);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
}  // namespace

extern "C" int mx_gemm_bf16_res_ln(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                                   const float* bias, const uint16_t* R, long ldr, uint16_t* X, long ldx,
                                   const uint16_t* gamma, const uint16_t* beta, uint16_t* Y, long ldy, int M, int N,
                                   int K, int Kw, float eps, uint64_t* stats, long stats_words, uint32_t* sync,
                                   long sync_words) {
  return launch_rln<1>(st, A, lda, W, ldw, bias, R, ldr, X, ldx, gamma, beta, Y, ldy, M, N, K, Kw, eps, stats,
                       stats_words, sync, sync_words);
}

// The same launch with the TRecViT RMSNorm instead of the LayerNorm (the epilogue of mx_residual_rmsnorm): Y =
// bf16(bf16(x' rstd) sc1), rstd = bf16(1 / sqrt(bf16(bf16(sum bf16(x'^2) / N) + eps))), sc1 = bf16(scale + 1). The
// tiles exchange their rows' sums of bf16(x'^2); stats / sync are the same words as mx_gemm_bf16_res_ln's (calls of
// either form with the same N may share them, ordered on one stream).
extern "C" int mx_gemm_bf16_res_rms(hipStream_t st, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                                    const float* bias, const uint16_t* R, long ldr, uint16_t* X, long ldx,
                                    const uint16_t* sc1, uint16_t* Y, long ldy, int M, int N, int K, int Kw, float eps,
                                    uint64_t* stats, long stats_words, uint32_t* sync, long sync_words) {
  return launch_rln<2>(st, A, lda, W, ldw, bias, R, ldr, X, ldx, sc1, nullptr, Y, ldy, M, N, K, Kw, eps, stats,
                       stats_words, sync, sync_words);
}
