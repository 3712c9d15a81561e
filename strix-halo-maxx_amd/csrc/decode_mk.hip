// One-launch greedy decode step for the moondream2 text model (24 layers, hidden 2048, 32 heads x 64, MLP 8192,
// vocab 51200): every layer, the LM head, the argmax and the next token's embedding in a single persistent kernel.
//
// Why: a decode step streams 2.6 GB of weights, ~100 MB per layer. As separate kernels (decode.hip) every layer pays
// three kernel boundaries, each a launch plus a dependent load -> compute -> store chain during which HBM idles
// (~9 us of a ~27 us layer). Here the boundaries become data-ready waits between workgroups, and each workgroup has
// already issued the weight rows (or K/V cache rows) of its next phase when it starts waiting, so HBM keeps
// streaming through every wait.
//
// Grid: 256 workgroups of 512 threads (8 waves), one per CU, all resident at once (the host checks the CU count).
//   * GEMV workgroups g = 0 .. 223, per layer:
//       A  h = LN(x) (each wave, from x in LDS), rows 64 g .. 64 g + 63 of [Wqkv | Wfc1] (8 rows per wave), + bias,
//          GELU (tanh) on the fc1 rows -> qkv / g exchange words
//       B  y2 = bf16(g W2^T + b2) for this workgroup's 8 or 10 fc2 rows (one row per wave, two on waves 0-1 of the
//          10-row groups), g gathered into LDS
//       C  x'[n] = bf16(y2[n] + bf16(bf16(a Wp^T + bp)[n] + x[n])) for the same rows (md2fast.py:198's parallel
//          residual, the roundings of decode.hip's gemv_res2), a gathered into LDS -> x exchange words
//   * attention workgroups 224 .. 255, one per head: during phase A they load the head's K / V cache rows
//     0 .. pos - 1 into registers (16 rounds of 8 keys per wave: contexts up to 1024), then wait for the head's q / k /
//     v, apply the rope (fp32, as rope.hip), append k / v at pos, and run a one-pass softmax over all keys (8 waves
//     merged in LDS) -> attention output words
//   * LM head (all 256 workgroups): LN(x) with the final LayerNorm, logits = bf16(x Wlm^T + b) in 8-row jobs, a
//     per-workgroup argmax key; workgroup 0 reduces the 256 keys (first index wins ties, as torch.argmax), records
//     the token, advances the position and writes the next token's embedding (embed_step_kernel's bookkeeping).
//
// Exchange: activation vectors travel as 64-bit words (epoch << 32 | two bf16), written with agent-scope stores and
// read with agent-scope loads (both bypass the non-coherent per-XCD L2), so a reader polls the data itself: a word
// with the expected epoch is the new value (8-byte stores are single-copy atomic). Epochs grow by 3 per layer within
// a step and the base advances by kEpochsPerStep per step (kept in device memory), so a buffer can be reused by every
// layer: no producer can overwrite a word before all of its readers have consumed it (each next write depends,
// through the phase chain, on every reader having finished). Every wait is bounded (~50 ms of the 100 MHz clock);
// a wait that times out records an error code and the workgroup exits, so the grid always drains.
#include "common.h"
#include "gemv.h"

namespace {

constexpr int MK_D = 2048, MK_H = 32, MK_HD = 64, MK_F = 8192;
constexpr int MK_NQKV = 3 * MK_D, MK_NA = MK_NQKV + MK_F;  // 6144 qkv rows + 8192 fc1 rows
constexpr int MK_W = 8, MK_T = 64 * MK_W;                   // waves / threads per workgroup
constexpr int MK_NG = 224, MK_G = MK_NG + MK_H;             // GEMV workgroups, all workgroups
constexpr int MK_RA = MK_NA / MK_NG;                         // 64 phase-A rows per GEMV workgroup
static_assert(MK_RA == 8 * MK_W, "8 rows per wave");
constexpr int MK_ROUNDS = 16;                                // key rounds of 8 keys per wave: 1024 keys
constexpr int MK_MAXKEYS = MK_ROUNDS * 8 * MK_W;

// exchange words (uint64): layout of the LL area
constexpr int LL_X = 0, LL_QKV = 1024, LL_G = 4096, LL_A = 8192, LL_AM = 9216, LL_WORDS = 9216 + MK_G;
constexpr uint64_t kTimeout = 5000000ull;  // 50 ms at 100 MHz

// fc2 / proj rows of GEMV workgroup g: 128 groups of 10 rows, then 96 of 8 (even sizes: pairs stay together)
__device__ __forceinline__ void row_group(int g, int& r0, int& n) {
  if (g < 128) r0 = 10 * g, n = 10;
  else r0 = 1280 + 8 * (g - 128), n = 8;
}

// Every pointer here is to device memory: the casts to the global address space keep the loads and stores global
// (pointers read from the layer table, or passed through the opaque asm below, would otherwise become flat accesses,
// which also count against the LDS wait counter).
#define GLOBAL(T, p) ((__attribute__((address_space(1))) T*)(p))

__device__ __forceinline__ void st_word(uint64_t* p, uint32_t ep, uint32_t payload) {
  __hip_atomic_store(GLOBAL(uint64_t, p), ((uint64_t)ep << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
  return __hip_atomic_load(GLOBAL(uint64_t, const_cast<uint64_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ldg(const T* p) { return *GLOBAL(const T, p); }
__device__ __forceinline__ u32x4 ldg_vec(const uint16_t* p) { return *GLOBAL(const u32x4, p); }
template <int KC>
__device__ __forceinline__ void load_vec_g(u32x4 (&xc)[KC], const uint16_t* x, int lane) {
#pragma unroll
  for (int i = 0; i < KC; i++) xc[i] = ldg_vec(x + (lane + 64 * i) * 8);
}

// Wait until words buf[0 .. NW) all carry epoch ep and store their payloads to dst[0 .. NW) (LDS). Every thread of
// the workgroup calls it; each round issues all of a thread's loads before checking any (one round trip per round;
// words already seen are simply read again). false: the wait timed out (error recorded); the caller returns.
template <int NW>
__device__ bool ll_gather(const uint64_t* __restrict__ buf, uint32_t ep, uint32_t* dst, uint32_t* err, int* s_flag) {
  constexpr int PER = (NW + MK_T - 1) / MK_T;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    uint64_t v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) v[i] = ld_word(buf + min((int)threadIdx.x + MK_T * i, NW - 1));
    int pending = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int w = threadIdx.x + MK_T * i;
      if (w < NW) {
        if ((uint32_t)(v[i] >> 32) == ep) dst[w] = (uint32_t)v[i];
        else pending = 1;
      }
    }
    if (!__syncthreads_or(pending)) return true;
    if (threadIdx.x == 0) *s_flag = (__builtin_amdgcn_s_memrealtime() - t0) > kTimeout;
    __syncthreads();
    if (*s_flag) {
      if (threadIdx.x == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

struct MkLayer {  // 10 device pointers, in this order (the host builds the table)
  const uint16_t *ln_g, *ln_b;  // LayerNorm (2048)
  const uint16_t* wqf;          // [6144 + 8192][2048]: qkv rows then fc1 rows
  const float* bqf;
  const uint16_t* w2;           // [2048][8192]
  const float* b2;
  const uint16_t* wp;           // [2048][2048]
  const float* bp;
  uint16_t *kc, *vc;            // [32][ctx][64] (cache slot 0)
};

struct MkArgs {
  const MkLayer* layers;
  int nl, ctx, V, pos_base, cap;
  float eps, scale_log2;
  const uint16_t *lnf_g, *lnf_b, *wlm;
  const float* blm;
  const uint16_t* wte;
  const float* cs;      // rope table [pos][32] (cos, sin pairs)
  uint16_t* x;          // the step's input embedding (2048); the next step's embedding is written here
  int* state;           // [0] tokens emitted, [1] position of the token in x
  int* tokens;
  uint16_t* logits;     // optional (V)
  uint64_t* ll;         // LL_WORDS exchange words
  uint32_t* ep;         // [0] epoch base, [1] error code (0 = none)
};

// 16-byte chunk of a weight matrix at byte offset off (32-bit) from a wave-uniform base: one offset register per
// row, the chunk steps as immediates (64-bit addresses per chunk, hoisted out of the layer loop, spilled)
__device__ __forceinline__ u32x4 ldw(const uint16_t* base, uint32_t off) {
  return __builtin_nontemporal_load(GLOBAL(const u32x4, reinterpret_cast<const char*>(base) + off));
}

constexpr int MK_MAXL = 32;  // layers the LDS copy of the layer table holds

// Layer l's descriptor from the LDS copy of the table, every pointer made wave-uniform (SGPRs): read from global memory
// inside the loop they would be vector loads, whose waits (in-order with the weight stream) would drain every
// prefetched weight row.
__device__ __forceinline__ MkLayer layer_of(const uint64_t* tab, int l) {
  uint64_t v[10];
#pragma unroll
  for (int i = 0; i < 10; i++) {
    const uint64_t t = tab[l * 10 + i];
    v[i] = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(t >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)t);
  }
  MkLayer L;
  __builtin_memcpy(&L, v, sizeof(L));
  return L;
}

__device__ __forceinline__ uint32_t amax_key32(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (u & 0xffff0000u) | (0xffffu - (uint32_t)idx);  // v is a bf16 value: its low 16 bits carry no order
}

__global__ __launch_bounds__(MK_T) void decode_mk_kernel(MkArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t xs[MK_D / 2];   // x: the layer's input (bf16 pairs)
  __shared__ __attribute__((aligned(16))) uint32_t gs[MK_F / 2];   // fc1 output g
  __shared__ __attribute__((aligned(16))) uint32_t as2[MK_D / 2];  // attention output
  __shared__ __attribute__((aligned(16))) uint16_t qkvh[3 * MK_HD]; // attention: the head's q, k, v (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t qr[MK_HD], kr[MK_HD];  // roped q, k (bf16)
  __shared__ float rec[MK_W][2 + MK_HD];
  __shared__ float ys[16];
  __shared__ uint32_t sbest[MK_W];
  __shared__ int s_flag;
  __shared__ uint64_t stab[MK_MAXL * 10];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
  for (int i = tid; i < a.nl * 10; i += MK_T) stab[i] = reinterpret_cast<const uint64_t*>(a.layers)[i];
  __syncthreads();
  const uint32_t base = a.ep[0];
  const int pos = min(max(a.state[1], 0), a.ctx - 1);
  const int NL = a.nl;
  auto E = [&](int l, int p) { return base + 3u * (uint32_t)l + (uint32_t)p; };
  uint32_t* err = a.ep + 1;

  if (wg >= MK_NG) {
    // ======================================================================= attention workgroup (one head)
    const int h = wg - MK_NG;
    const int sub = lane & 7, kg = lane >> 3;
    const int kmax = max(pos - 1, 0);  // last cache row (rows 0 .. pos - 1 hold earlier tokens)
    for (int l = 0; l < NL; l++) {
      const MkLayer L = layer_of(stab, l);
      uint32_t so = (uint32_t)sub * 8u;  // opaque: addresses rebuilt per layer, not hoisted (they would spill)
      asm volatile("" : "+v"(so));
      uint64_t* ll = a.ll;
      asm volatile("" : "+s"(ll));
      const uint16_t* kh = L.kc + (long)h * a.ctx * MK_HD;
      const uint16_t* vh = L.vc + (long)h * a.ctx * MK_HD;
      // the head's cache rows, issued before the wait for q / k / v (32-bit offsets from the head's base)
      u32x4 kk[MK_ROUNDS], vv[MK_ROUNDS];
#pragma unroll
      for (int r = 0; r < MK_ROUNDS; r++) {
        const int key = min(wave * 8 + kg + 64 * r, kmax);
        const unsigned off = (unsigned)key * 64u + so;
        kk[r] = ldg_vec(kh + off);
        vv[r] = ldg_vec(vh + off);
      }
      // q, k, v of the head (96 words: q at h * 32, k at 1024 + h * 32, v at 2048 + h * 32); the wait also completes
      // the cache loads above
      {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        const int w = (min(tid, 95) >> 5) * 1024 + h * 32 + (tid & 31);
        for (;;) {
          const uint64_t v = ld_word(ll + LL_QKV + w);
          int pending = 0;
          if (tid < 96) {
            if ((uint32_t)(v >> 32) == E(l, 1)) reinterpret_cast<uint32_t*>(qkvh)[tid] = (uint32_t)v;
            else pending = 1;
          }
          if (!__syncthreads_or(pending)) break;
          if (tid == 0) s_flag = (__builtin_amdgcn_s_memrealtime() - t0) > kTimeout;
          __syncthreads();
          if (s_flag) {
            if (tid == 0) __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
          }
        }
      }
      // rope of the new token's q and k (fp32, rope.hip's arithmetic): output dim d < 32 pairs input dims
      // (d >> 1, 16 + (d >> 1)); the roped k and the raw v are appended at pos after the last barrier of the layer
      uint16_t kapp = 0, vapp = 0;
      if (tid < MK_HD) {
        const int d = tid, jr = (d & 31) >> 1;
        const float* cp = a.cs + (long)pos * 32;
        const float cr = ldg(cp + 2 * jr), sr = ldg(cp + 2 * jr + 1);
        const int d0 = d < 32 ? jr : d;
        const float qa = bf2f(qkvh[d0]), qb = bf2f(qkvh[16 + jr]);
        const float ka = bf2f(qkvh[MK_HD + d0]), kb = bf2f(qkvh[MK_HD + 16 + jr]);
        const float qo = __fadd_rn(__fmul_rn(qa, sr), __fmul_rn(qb, cr)), qe = __fsub_rn(__fmul_rn(qa, cr), __fmul_rn(qb, sr));
        const float ko = __fadd_rn(__fmul_rn(ka, sr), __fmul_rn(kb, cr)), ke = __fsub_rn(__fmul_rn(ka, cr), __fmul_rn(kb, sr));
        const float qv = d < 32 ? ((d & 1) ? qo : qe) : qa;
        const float kv = d < 32 ? ((d & 1) ? ko : ke) : ka;
        qr[d] = f2bf(qv);
        kapp = f2bf(kv);
        kr[d] = kapp;
        vapp = qkvh[2 * MK_HD + d];
      }
      __syncthreads();
      const u32x4 qp = *reinterpret_cast<const u32x4*>(&qr[sub * 8]);
      const u32x4 knew = *reinterpret_cast<const u32x4*>(&kr[sub * 8]);
      const u32x4 vnew = *reinterpret_cast<const u32x4*>(&qkvh[2 * MK_HD + sub * 8]);
      const u32x4 zero4 = {0u, 0u, 0u, 0u};
      // one pass over all keys 0 .. pos: scores (8 lanes per key), wave max, exponentials, P V
      float sv[MK_ROUNDS];
      float mb = -INFINITY;
#pragma unroll
      for (int r = 0; r < MK_ROUNDS; r++) {
        const int key = wave * 8 + kg + 64 * r;
        if (key == pos) { kk[r] = knew; vv[r] = vnew; }
        else if (key > pos) { kk[r] = zero4; vv[r] = zero4; }
        float sc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          sc = __builtin_fmaf(lo_bf(kk[r][e]), lo_bf(qp[e]), sc);
          sc = __builtin_fmaf(hi_bf(kk[r][e]), hi_bf(qp[e]), sc);
        }
        sc += __shfl_xor(sc, 1, 64);
        sc += __shfl_xor(sc, 2, 64);
        sc += __shfl_xor(sc, 4, 64);
        sc = key <= pos ? sc * a.scale_log2 : -INFINITY;
        sv[r] = sc;
        mb = fmaxf(mb, sc);
      }
      const float m = fmaxf(wave_max(mb), -1e30f);  // a wave whose keys are all past pos: p = 0, not NaN
      float lsum = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < MK_ROUNDS; r++) {
        const float pr = rbf(__builtin_amdgcn_exp2f(sv[r] - m));
        if (sub == 0) lsum += pr;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          o[2 * e] = __builtin_fmaf(pr, lo_bf(vv[r][e]), o[2 * e]);
          o[2 * e + 1] = __builtin_fmaf(pr, hi_bf(vv[r][e]), o[2 * e + 1]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        o[e] += __shfl_xor(o[e], 8, 64);
        o[e] += __shfl_xor(o[e], 16, 64);
        o[e] += __shfl_xor(o[e], 32, 64);
      }
      lsum = wave_sum(lsum);
      if (kg == 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) rec[wave][2 + sub * 8 + e] = o[e];
      }
      if (lane == 0) { rec[wave][0] = m; rec[wave][1] = lsum; }
      __syncthreads();
      if (tid < MK_HD / 2) {  // two output dims per thread -> one word
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < MK_W; w++) M = fmaxf(M, rec[w][0]);
        float Lt = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int w = 0; w < MK_W; w++) {
          const float f = __builtin_amdgcn_exp2f(rec[w][0] - M);
          Lt += rec[w][1] * f;
          a0 += rec[w][2 + 2 * tid] * f;
          a1 += rec[w][3 + 2 * tid] * f;
        }
        st_word(ll + LL_A + h * 32 + tid, E(l, 2), pack2(a0 / Lt, a1 / Lt));
      }
      if (tid < MK_HD) {  // the append (read by later steps only)
        *GLOBAL(uint16_t, L.kc + ((long)h * a.ctx + pos) * MK_HD + tid) = kapp;
        *GLOBAL(uint16_t, L.vc + ((long)h * a.ctx + pos) * MK_HD + tid) = vapp;
      }
      // no barrier here: rec, qkvh, qr, kr are next written after the next layer's q / k / v wait, which every
      // thread reaches only after its reads above (a barrier would also wait for the stores just issued)
    }
  } else {
    // ======================================================================= GEMV workgroup
    int r0, nr;
    row_group(wg, r0, nr);
    const int gw = wg * MK_W + wave;  // 1792 GEMV waves; phase-A job j covers rows j * 7168 + 4 gw .. + 3
    u32x4 wa[4][4];                   // one 4-row phase-A job in flight
    auto issue_a = [&](const MkLayer& L, uint32_t lo, int j) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t o = (uint32_t)(j * 7168 + 4 * gw + r) * (MK_D * 2u) + lo;
#pragma unroll
        for (int i = 0; i < 4; i++) wa[r][i] = ldw(L.wqf, o + 1024u * i);
      }
    };
    {
      uint32_t lo = (uint32_t)lane * 16u;
      asm volatile("" : "+v"(lo));
      issue_a(layer_of(stab, 0), lo, 0);
    }
    for (int l = 0; l < NL; l++) {
      const MkLayer L = layer_of(stab, l);
      // the lane's byte offset, opaque to the compiler: the addresses derived from it are rebuilt every layer instead
      // of being hoisted out of the loop (live across it, they spill; a spill reload waits for every load before it)
      uint32_t lo = (uint32_t)lane * 16u;
      asm volatile("" : "+v"(lo));
      uint64_t* ll = a.ll;  // the exchange addresses likewise
      asm volatile("" : "+s"(ll));
      // ---- phase A: LN(x), then two 4-row jobs of [Wqkv | Wfc1] (job 0 was issued before the wait for x; job 0 of
      // every wave together covers all qkv rows, so the attention can start after the first job)
      u32x4 gc[4], bc[4];
      load_vec_g<4>(gc, L.ln_g, lane);
      load_vec_g<4>(bc, L.ln_b, lane);
      if (l == 0) {
        for (int i = tid; i < MK_D / 8; i += MK_T)
          reinterpret_cast<u32x4*>(xs)[i] = ldg_vec(a.x + i * 8);
        __syncthreads();
      } else if (!ll_gather<MK_D / 2>(ll + LL_X, E(l - 1, 3), xs, err, &s_flag)) {
        return;
      }
      u32x4 xc[4];
      load_vec<4>(xc, reinterpret_cast<const uint16_t*>(xs), lane);
      ln_chunks<4>(xc, gc, bc, a.eps, MK_D, lane);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        float acc[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          acc[r] = 0.f;
#pragma unroll
          for (int i = 0; i < 4; i++) acc[r] = dot8(wa[r][i], xc[i], acc[r]);
        }
        __builtin_amdgcn_sched_barrier(0);  // job 0's registers are free before job 1's loads land in them
        if (j == 0) issue_a(L, lo, 1);
        const int row = j * 7168 + 4 * gw + (lane >> 4);
        const float bme = ldg(L.bqf + row);
        const float tot = reduce_rows<4>(acc, lane);  // lane l: row 4 gw + (l >> 4) of the job
        float v = rbf(tot + bme);
        if (row >= MK_NQKV) v = rbf(gelu_tanh(v));
        const float vn = __shfl_down(v, 16, 64);  // the odd row of the pair
        if ((lane & 31) == 0) {
          const uint32_t w = pack2(v, vn);
          if (row < MK_NQKV) st_word(ll + LL_QKV + row / 2, E(l, 1), w);
          else st_word(ll + LL_G + (row - MK_NQKV) / 2, E(l, 1), w);
        }
      }
      // ---- phase B: fc2 rows r0 + wave (and r0 + 8 + wave on waves 0-1 of 10-row groups): the first row issued
      // before the wait for g, the second after it
      const bool two = wave + 8 < nr;
      const int n1 = r0 + wave, n2 = two ? r0 + 8 + wave : n1;
      __builtin_amdgcn_sched_barrier(0);
      u32x4 w2[16];
      const uint32_t o2a = (uint32_t)n1 * (MK_F * 2u) + lo;
#pragma unroll
      for (int i = 0; i < 16; i++) w2[i] = ldw(L.w2, o2a + 1024u * i);
      if (!ll_gather<MK_F / 2>(ll + LL_G, E(l, 1), gs, err, &s_flag)) return;
      float y2a, y2b = 0.f;
      {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) acc = dot8(w2[i], *reinterpret_cast<const u32x4*>(&gs[(lane + 64 * i) * 4]), acc);
        y2a = rbf(wave_sum(acc) + ldg(L.b2 + n1));
      }
      __builtin_amdgcn_sched_barrier(0);
      if (two) {  // wave-uniform
        const uint32_t o2b = (uint32_t)n2 * (MK_F * 2u) + lo;
#pragma unroll
        for (int i = 0; i < 16; i++) w2[i] = ldw(L.w2, o2b + 1024u * i);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) acc = dot8(w2[i], *reinterpret_cast<const u32x4*>(&gs[(lane + 64 * i) * 4]), acc);
        y2b = rbf(wave_sum(acc) + ldg(L.b2 + n2));
      }
      // ---- phase C: proj rows n1 (, n2), issued before the wait for the attention output
      __builtin_amdgcn_sched_barrier(0);
      u32x4 wpa[4], wpb[4];
      const uint32_t opa = (uint32_t)n1 * (MK_D * 2u) + lo;
      const uint32_t opb = (uint32_t)n2 * (MK_D * 2u) + lo;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        wpa[i] = ldw(L.wp, opa + 1024u * i);
        wpb[i] = ldw(L.wp, opb + 1024u * i);  // n2 == n1 on one-row waves: the same (cached) row
      }
      const float bpa = ldg(L.bp + n1), bpb = ldg(L.bp + n2);
      if (!ll_gather<MK_D / 2>(ll + LL_A, E(l, 2), as2, err, &s_flag)) return;
      {
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 av = *reinterpret_cast<const u32x4*>(&as2[(lane + 64 * i) * 4]);
          acc[0] = dot8(wpa[i], av, acc[0]);
          acc[1] = dot8(wpb[i], av, acc[1]);
        }
        const float ta = wave_sum(acc[0]), tb = wave_sum(acc[1]);
        const uint16_t* xb = reinterpret_cast<const uint16_t*>(xs);
        if (lane == 0) {
          ys[wave] = rbf(y2a + rbf(rbf(ta + bpa) + bf2f(xb[n1])));
          if (two) ys[8 + wave] = rbf(y2b + rbf(rbf(tb + bpb) + bf2f(xb[n2])));
        }
      }
      __syncthreads();
      if (tid < nr / 2) {
        // rows r0 + 2 tid, r0 + 2 tid + 1: staged at index (row - r0)
        st_word(ll + LL_X + r0 / 2 + tid, E(l, 3), pack2(ys[2 * tid], ys[2 * tid + 1]));
      }
      // the next layer's first phase-A job, in flight during the wait for x (ys is rewritten only after that wait)
      __builtin_amdgcn_sched_barrier(0);
      if (l + 1 < NL) issue_a(layer_of(stab, l + 1), lo, 0);
    }
  }

  // ========================================================================= LM head + argmax (all workgroups)
  {
    const int gw = wg * MK_W + wave;  // 2048 waves; 4-row jobs gw, gw + 2048, ...
    const int njobs = (a.V + 3) / 4;
    uint32_t lo = (uint32_t)lane * 16u;
    asm volatile("" : "+v"(lo));
    uint64_t* ll = a.ll;
    asm volatile("" : "+s"(ll));
    u32x4 gc[4], bc[4];
    load_vec<4>(gc, a.lnf_g, lane);
    load_vec<4>(bc, a.lnf_b, lane);
    typedef u32x4 Job[4][4];
    Job wv0, wv1;  // two 4-row jobs: the next one in flight while one is reduced (static names: no scratch)
    auto issue = [&](int j, Job& w) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t o = (uint32_t)min(4 * j + r, a.V - 1) * (MK_D * 2u) + lo;
#pragma unroll
        for (int i = 0; i < 4; i++) w[r][i] = ldw(a.wlm, o + 1024u * i);
      }
    };
    uint32_t best = 0u;
    u32x4 xc[4];
    auto reduce_job = [&](int j, const Job& w) {
      float acc[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        acc[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r] = dot8(w[r][i], xc[i], acc[r]);
      }
      const int n = 4 * j + (lane >> 4);
      const float bme = a.blm[min(n, a.V - 1)];
      const float tot = reduce_rows<4>(acc, lane);
      if (n < a.V) {
        const float v = rbf(tot + bme);
        if (a.logits && (lane & 15) == 0) a.logits[n] = f2bf(v);
        const uint32_t k = amax_key32(v, n);
        best = k > best ? k : best;
      }
    };
    constexpr int SJ = MK_G * MK_W;
    if (gw < njobs) issue(gw, wv0);
    if (!ll_gather<MK_D / 2>(ll + LL_X, E(NL - 1, 3), xs, err, &s_flag)) return;
    load_vec<4>(xc, reinterpret_cast<const uint16_t*>(xs), lane);
    ln_chunks<4>(xc, gc, bc, a.eps, MK_D, lane);
    for (int j = gw; j < njobs; j += 2 * SJ) {
      if (j + SJ < njobs) issue(j + SJ, wv1);
      reduce_job(j, wv0);
      if (j + SJ < njobs) {
        if (j + 2 * SJ < njobs) issue(j + 2 * SJ, wv0);
        reduce_job(j + SJ, wv1);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t t = __shfl_xor(best, o, 64);
      best = t > best ? t : best;
    }
    if (lane == 0) sbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
      uint32_t b = sbest[0];
#pragma unroll
      for (int w = 1; w < MK_W; w++) b = sbest[w] > b ? sbest[w] : b;
      st_word(ll + LL_AM + wg, base + 3u * (uint32_t)NL + 1u, b);
    }
  }
  if (wg != 0) return;
  // ---- workgroup 0: the token, the bookkeeping of embed_step_kernel, the next embedding, the next epoch base
  if (!ll_gather<MK_G>(a.ll + LL_AM, base + 3u * (uint32_t)NL + 1u, xs, err, &s_flag)) return;
  if (tid < 64) {
    uint32_t b = 0u;
    for (int i = tid; i < MK_G; i += 64) b = xs[i] > b ? xs[i] : b;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t t = __shfl_xor(b, o, 64);
      b = t > b ? t : b;
    }
    if (tid == 0) sbest[0] = b;
  }
  __syncthreads();
  const int tok = min((int)(0xffffu - (sbest[0] & 0xffffu)), a.V - 1);
  if (tid == 0) {
    const int s = a.state[0];
    if (s < a.cap) {
      a.tokens[s] = tok;
      a.state[1] = a.pos_base + s;
      a.state[0] = s + 1;
    }
    a.ep[0] = base + 3u * (uint32_t)NL + 2u;
  }
  for (int i = tid; i < MK_D / 8; i += MK_T)
    *reinterpret_cast<u32x4*>(a.x + i * 8) = *reinterpret_cast<const u32x4*>(a.wte + (long)tok * MK_D + i * 8);
}

}  // namespace

extern "C" int mx_decode_mk_words(void) { return LL_WORDS; }

extern "C" int mx_decode_mk_grid(void) { return MK_G; }

// One greedy decode step of the 2048-wide, 32-head text model in one launch (decode_mk_kernel): layers[nl] describes
// every layer's weights and cache (device memory), x the step's input embedding (replaced by the next step's), state /
// tokens / cap / pos_base as mx_embed_step; logits optional (V bf16). ll: mx_decode_mk_words() zeroed words, ep: 2
// words {epoch base, error} zeroed once, both owned by one decoder (the kernel advances the base). Needs
// mx_decode_mk_grid() CUs (one workgroup on each, all resident) and ctx <= 1024 (the keys one pass holds).
extern "C" int mx_decode_step_mk(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g,
                                 const uint16_t* lnf_b, const uint16_t* wlm, const float* blm, int V,
                                 const uint16_t* wte, const float* cs, float eps, float scale, uint16_t* x, int* state,
                                 int pos_base, int* tokens, int cap, uint16_t* logits, uint64_t* ll, uint32_t* ep) {
  if (!layers || !lnf_g || !lnf_b || !wlm || !blm || !wte || !cs || !x || !state || !tokens || !ll || !ep)
    return MX_ENULL;
  if (nl < 1 || nl > MK_MAXL || ctx < 1 || ctx > MK_MAXKEYS || V < 1 || V > 65536 || cap < 1 || pos_base < 0)
    return MX_ESHAPE;
  if (((uintptr_t)x | (uintptr_t)wlm | (uintptr_t)wte) & 15) return MX_ELAYOUT;
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return MX_ELAUNCH;
  if (ncu < MK_G) return MX_ESHAPE;  // every workgroup must be resident at once
  MkArgs a;
  a.layers = static_cast<const MkLayer*>(layers);
  a.nl = nl, a.ctx = ctx, a.V = V, a.pos_base = pos_base, a.cap = cap;
  a.eps = eps, a.scale_log2 = scale * 1.4426950408889634f;
  a.lnf_g = lnf_g, a.lnf_b = lnf_b, a.wlm = wlm, a.blm = blm, a.wte = wte, a.cs = cs;
  a.x = x, a.state = state, a.tokens = tokens, a.logits = logits, a.ll = ll, a.ep = ep;
  hipLaunchKernelGGL(decode_mk_kernel, dim3(MK_G), dim3(MK_T), 0, st, a);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Bytes of one layer descriptor in the layers array of mx_decode_step_mk: 10 device pointers (ln_g, ln_b, wqf, bqf,
// w2, b2, wp, bp, kc, vc), in that order, 8 bytes each.
extern "C" int mx_decode_mk_layer_bytes(void) { return (int)sizeof(MkLayer); }
