// One-launch greedy decode step for the moondream2 text model (24 layers, hidden 2048, 32 heads x 64, MLP 8192,
// vocab 51200): every layer, the LM head, the argmax and the next token's embedding in a single persistent kernel.
//
// Why: a decode step streams 2.6 GB of weights, ~100 MB per layer. As separate kernels (decode.hip) every layer pays
// three kernel boundaries, each a launch plus a dependent load -> compute -> store chain during which HBM idles
// (~9 us of a ~27 us layer). Here the boundaries become data-ready waits between workgroups, and the weight stream
// never stops for them.
//
// Grid: 256 workgroups of 9 waves, one per CU, all resident at once (the host checks the CU count). In every
// workgroup waves 0-7 compute and wave 8 is the exchange wave: it alone waits for other workgroups' results (polls)
// and publishes most of this workgroup's. Vector-memory completion is in order per wave, so a wave that polled would
// first wait for every weight row it has in flight; the compute waves never poll and meet the exchange wave at plain
// s_barriers (no memory wait), so each keeps its next rows in flight through every exchange.
//   * GEMV workgroups g = 0 .. 223, per layer (compute wave w):
//       the exchange wave gathers x and computes h = LN(x) into LDS (the proj rows of the workgroup arrive in LDS by
//          DMA meanwhile)
//       A  [Wqkv | Wfc1] in row pairs: pair round k gives each wave one pair (qkv pairs in the first rounds), each row
//          + bias, GELU (tanh) on fc1 rows -> qkv / g exchange words, stored in two bursts
//       B  the 8 or 10 fc2 rows of the workgroup in 4 KB quarter rows, spread over the waves -> partial sums in LDS
//       C  the same proj rows from LDS -> partial sums; the exchange wave then forms
//          x'[n] = bf16(y2[n] + bf16(bf16(a Wp^T + bp)[n] + x[n])), y2 = bf16(g W2^T + b2) (md2fast.py:198's
//          parallel residual, the roundings of decode.hip's gemv_res2) -> x exchange words
//     Each compute wave streams A and B through a ring of MK_NB 4 KB units (the next unit issued as soon as one is
//     reduced, across phase and layer boundaries).
//   * attention workgroups 224 .. 255, one per head: the compute waves load the head's K cache rows 0 .. pos - 1
//     into registers and its V rows into LDS (LDS-DMA), 8 keys per wave per round, 16 rounds (contexts up to 1024),
//     as soon as the previous layer's attention is done; the exchange wave waits for the head's q / k / v, applies
//     the rope (fp32, as rope.hip), and after the compute waves' one-pass softmax (merged in LDS) publishes the
//     output and appends k / v at pos.
//   * LM head (all 256 workgroups): LN(x) with the final LayerNorm, logits = bf16(x Wlm^T + b) in 2-row jobs, a
//     per-workgroup argmax key; workgroup 0 reduces the 256 keys (first index wins ties, as torch.argmax), records
//     the token, advances the position and writes the next token's embedding (embed_step_kernel's bookkeeping).
//
// What bounds it (measured): every exchange waits behind the requests queued ahead of it in the memory system, so the
// kernel keeps the queue short (~64 KB per CU in flight: the ring, no deeper) and keeps polls off the weight stream
// (the exchange wave polls for g only once its own phase A is done; one sentinel per 64 words, then one batch read).
// Exchange: activation vectors travel as 64-bit words (epoch << 32 | two bf16), written with agent-scope stores and
// read with agent-scope loads (both bypass the non-coherent per-XCD L2), so a reader polls the data itself: a word
// with the expected epoch is the new value (8-byte stores are single-copy atomic). Epochs grow by 3 per layer within
// a step and the base advances by 3 L + 2 per step (kept in device memory), so a buffer is reused by every layer: no
// producer can overwrite a word before all of its readers have consumed it (each next write depends, through the
// phase chain, on every reader having finished). An exchange wave polls one word per 64 until they all carry the
// epoch, then reads the whole vector (again where a word is still stale). Every wait is bounded (~50 ms of the
// 100 MHz clock): after a timeout the exchange wave records an error code and stops waiting, so every wave still
// reaches every barrier and the grid drains (the step's results are then garbage; the host sees the code).
#include "common.h"
#include "gemv.h"

#include <utility>

namespace {

constexpr int MK_D = 2048, MK_H = 32, MK_HD = 64, MK_F = 8192;
constexpr int MK_NQKV = 3 * MK_D, MK_NA = MK_NQKV + MK_F;  // 6144 qkv rows + 8192 fc1 rows
constexpr int MK_W = 8;                                     // compute waves per workgroup
constexpr int MK_XW = MK_W;                                 // the exchange wave
constexpr int MK_T = 64 * (MK_W + 1);                       // 576 threads
constexpr int MK_NG = 224, MK_G = MK_NG + MK_H;             // GEMV workgroups, all workgroups
#ifndef MK_GW
#define MK_GW 8
#endif
#ifndef MK_NB
#define MK_NB 5
#endif
// GEMV waves stream 4 KB weight units through a ring of MK_NB register buffers. Within a layer a unit is issued only
// MK_DIST = 2 slots ahead (~64 KB per CU in flight, about what saturates HBM, and no more): requests wait behind
// everything queued ahead of them, the exchanges between workgroups included, and with 128 KB per CU in flight a
// store -> poll round trip takes ~6 us instead of ~3, for no more bandwidth. At the end of a layer, where the next
// one can only start after the exchange of x, the whole ring is filled with the next layer's first units (MK_PF), so
// that the stream does not restart from empty. (MK_GW < 8 runs the GEMV on fewer waves, the others only meet the
// barriers.) Measured, steps per second: ring 2/2/2 1940, 3/2/3 2009, 4/2/4 2058, 5/2/5 2119, 6/2/6 2099, 4/3/4 1887.
constexpr int GW = MK_GW, NBUF = MK_NB;
#ifndef MK_DIST
#define MK_DIST 2
#endif
#ifndef MK_PF
#define MK_PF MK_NB
#endif
// Within a layer a unit is issued DIST slots ahead of its use; the first PF units of a layer are issued before its h
// barrier, at the end of the previous layer (any others up to DIST right after the barrier).
constexpr int DIST = MK_DIST, PF = MK_PF;
static_assert(DIST >= 1 && DIST <= NBUF && PF >= 0 && PF <= NBUF, "issue distances within the ring");
constexpr int MK_NGW = MK_NG * GW;                          // GEMV waves
constexpr int KA = (MK_NA / 2) / MK_NGW;                    // row pairs per GEMV wave in phase A
static_assert(KA * MK_NGW * 2 == MK_NA, "whole row pairs per wave");
constexpr int MK_RW = 8;                                    // fc2 / proj rows per workgroup (all 256)
static_assert(MK_RW * MK_G == MK_D, "the rows split evenly over the workgroups");
constexpr int JB = (4 * MK_RW + GW - 1) / GW;               // fc2 quarter-row units per wave
constexpr int JC = (MK_RW + GW - 1) / GW;                   // proj rows per wave
constexpr int JBA = 4 * MK_RW / MK_W, JCA = MK_RW / MK_W;   // the same in attention workgroups (all 8 waves)
static_assert(JBA == 4 && JCA == 1, "an attention-workgroup wave takes one whole fc2 row and one proj row");
// Slots of the weight ring: [0, SA) phase A, [B0, B1) phase B. Phase B is split at the middle of fc2's inputs: its
// first half [B0, BH) needs g[0, 4096) only, the second [BH, B1) g[4096, 8192). The first half of g is complete a
// pair round before the end of phase A, so the wait for the second half runs while the first half of B streams.
// Phase C's proj rows go to LDS by DMA at the start of the layer instead (C runs last, when the attention output
// arrives: rows fetched into the ring only then would add a memory latency to every layer).
static_assert(JB % 2 == 0, "B splits into two halves");
// The same ring for the W8A8 form (the reference's default text path: int8 weight rows with fp32 per-row scales,
// activations quantised per token): a 4 KB unit is then a phase-A row pair or half an fc2 row, and phase B cannot be
// split (g's quantisation scale is its maximum over all 8192 values).
template <bool I8>
struct RingCfg {
  static constexpr int SA = I8 ? KA : 2 * KA;                 // phase-A slots
  static constexpr int NB = I8 ? 2 * MK_RW / GW : JB;          // phase-B units per wave
  static constexpr int B0 = SA, B1 = SA + NB, BH = I8 ? B0 : B0 + NB / 2;
  static constexpr int NSLOT = (B1 + NBUF - 1) / NBUF * NBUF;  // slots per layer (a multiple of the ring depth)
};
static_assert(2 * MK_RW % GW == 0, "whole int8 fc2 half rows per wave");
static_assert(GW == 8, "the W8A8 form quantises with every wave of the workgroup: no idle waves");
// Barriers per layer: h ready, phase A done, g1 ready, g2 ready, a ready, partial sums ready (attention workgroups:
// q / k / v ready and the softmax merged instead of the first two). The exchange wave polls for g only once its own
// workgroup's phase A is done: 224 workgroups polling 64 sentinels each slow the weight stream of phase A down (the
// polls share each CU's memory pipeline), and g cannot be complete earlier anyway.
constexpr int NBAR = 6;
#ifndef MK_ROT
#define MK_ROT 1
#endif
// Row blocks rotate over the 8 workgroups of each group of 8 (consecutive workgroups sit on the 8 XCDs) from one
// phase-A pair round to the next, so that every XCD reads every part of the address interleave: with a fixed
// assignment, the XCDs whose blocks fall on some address bits stream up to 1.5x slower than the others, and every
// workgroup waits for the slowest.
constexpr int ROT = MK_ROT ? 8 / KA > 0 ? 8 / KA : 1 : 0;
constexpr int KQ = (MK_NQKV / 2 + MK_NGW - 1) / MK_NGW - 1;  // the last pair round that holds qkv pairs
constexpr int KG1 = (MK_NQKV / 2 + MK_F / 4 + MK_NGW - 1) / MK_NGW - 1;  // ... that holds pairs of g[0, 4096)
static_assert(KQ < KG1 && KG1 < KA - 1, "three bursts");
// fc2 unit j of a wave: half j / (JB / 2) of the inputs, row wave + GW (i / 2) and quarter 2 half + (i & 1) of it
// (i = j % (JB / 2)): each wave takes whole rows, their first two quarters in B's first half
__device__ __forceinline__ int b_row(int wave, int j) { return wave + GW * ((j % (JB / 2)) >> 1); }
__device__ __forceinline__ int b_quarter(int j) { return 2 * (j / (JB / 2)) + (j & 1); }
// the GEMV wave whose row pairs workgroup wg's wave takes in pair round k
__device__ __forceinline__ int rot_wave(int wg, int wave, int k) { return ((wg & ~7) + ((wg + ROT * k) & 7)) * GW + wave; }
constexpr int MK_ROUNDS = 16;                               // key rounds of 8 keys per compute wave: 1024 keys
constexpr int MK_MAXKEYS = MK_ROUNDS * 8 * MK_W;
constexpr int MK_MAXL = 32;                                 // layers the LDS copy of the layer table holds
constexpr int MK_LP = 13;                                   // pointers per layer descriptor

// exchange words (uint64): layout of the LL area
constexpr int LL_X = 0, LL_QKV = 1024, LL_G = 4096, LL_A = 8192, LL_AM = 9216, LL_WORDS = 9216 + MK_G;
static_assert(LL_G == LL_QKV + MK_NQKV / 2, "g words follow the qkv words: pair p of [qkv | fc1] is word LL_QKV + p");
constexpr uint64_t kTimeout = 5000000ull;  // 50 ms at 100 MHz

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
// 16-byte chunk of a weight matrix at byte offset off (32-bit) from a wave-uniform base: one offset register per
// row, the chunk steps as immediates
__device__ __forceinline__ u32x4 ldw(const uint16_t* base, uint32_t off) {
  return __builtin_nontemporal_load(GLOBAL(const u32x4, reinterpret_cast<const char*>(base) + off));
}

// Workgroup barrier without __syncthreads' memory wait: only this wave's LDS accesses complete first, so the rows a
// compute wave has in flight stay in flight across it.
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// fc2 / proj rows of workgroup g: 8 each, the attention workgroups included (they finish their head before the fc2
// rows can start, and 2048 rows over the 224 GEMV workgroups alone would leave some with 10 rows, others with 8)
__device__ __forceinline__ void row_group(int g, int& r0, int& n) {
  r0 = MK_RW * g;
  n = MK_RW;
}

struct MkLayer {  // 13 device pointers, in this order (the host builds the table)
  const uint16_t *ln_g, *ln_b;  // LayerNorm (2048)
  const uint16_t* wqf;          // [6144 + 8192][2048]: qkv rows then fc1 rows (int8 in the W8A8 form)
  const float* bqf;
  const uint16_t* w2;           // [2048][8192] (int8)
  const float* b2;
  const uint16_t* wp;           // [2048][2048] (int8)
  const float* bp;
  uint16_t *kc, *vc;            // [32][ctx][64] (cache slot 0)
  const float *sqf, *sw2, *swp; // W8A8: per-row weight scales of wqf, w2, wp (unused in the bf16 form)
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

// Layer l's descriptor from the LDS copy of the table, every pointer made wave-uniform (SGPRs): read from global memory
// inside the loop they would be vector loads, whose waits (in order with the weight stream) would drain it.
__device__ __forceinline__ MkLayer layer_of(const uint64_t* tab, int l) {
  uint64_t v[MK_LP];
#pragma unroll
  for (int i = 0; i < MK_LP; i++) {
    const uint64_t t = tab[l * MK_LP + i];
    v[i] = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(t >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)t);
  }
  MkLayer L;
  __builtin_memcpy(&L, v, sizeof(L));
  return L;
}

// Dot product of 8 bf16 pairs (one 16-byte chunk of a weight row and of the activation) accumulated into acc with
// v_dot2_f32_bf16 (two products per instruction, straight from the packed operands: no conversions to hold in
// registers). The bf16 products are exact in fp32; only the accumulation order differs from a sequential FMA chain.
// (The components go through plain temporaries: __builtin_bit_cast applied to a vector component directly, w[e],
// compiles to component 0 for every e with this compiler.)
__device__ __forceinline__ float dot8d(u32x4 w, u32x4 x, float acc) {
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t we = w[e], xe = x[e];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, we), __builtin_bit_cast(bf16x2, xe), acc, false);
  }
  return acc;
}

// 16 int8 x int8 products (one 16-byte chunk of a weight row and of the quantised activation), added to acc exactly.
typedef int i32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int dot16_i8(u32x4 a, u32x4 w, int acc) {
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t ae = a[e], we = w[e];
    acc = __builtin_amdgcn_sdot4((int)ae, (int)we, acc, false);
  }
  return acc;
}
// Exact int32 sum over the wave (the DPP pattern of wave_total), returned wave-uniform.
__device__ __forceinline__ int wave_total_i(int v) {
  auto mv = [](int old, int x, auto ctrl, auto rm) __attribute__((always_inline)) {
    return __builtin_amdgcn_update_dpp(old, x, decltype(ctrl)::value, decltype(rm)::value, 0xf, false);
  };
  using std::integral_constant;
  v += mv(0, v, integral_constant<int, 0xb1>{}, integral_constant<int, 0xf>{});
  v += mv(0, v, integral_constant<int, 0x4e>{}, integral_constant<int, 0xf>{});
  v += mv(0, v, integral_constant<int, 0x141>{}, integral_constant<int, 0xf>{});
  v += mv(0, v, integral_constant<int, 0x140>{}, integral_constant<int, 0xf>{});
  v += mv(0, v, integral_constant<int, 0x142>{}, integral_constant<int, 0xa>{});
  v += mv(0, v, integral_constant<int, 0x143>{}, integral_constant<int, 0xc>{});
  return __builtin_amdgcn_readlane(v, 63);
}
// Per-token int8 quantisation of a bf16 vector: s = max(max |x|, 1e-5) / 127, q = trunc(x / s + 0.5 sign) with the
// IEEE quotient (tgemm.py:81-91 _quant_rows, decode.hip's quant_vals_block_i8). The quotient is taken as x * (1 / s),
// within 1.5e-5 of x / s for |x / s| <= 127 (two roundings of 2^-24 relative); only where |t| + 0.5 lies within 1e-4
// of an integer could that change the truncated result, and there the exact quotient decides. The q values are those
// of the IEEE division.
// 8 values of a bf16 chunk quantised with scale s (rs = 1 / s) into two words; near: set where the multiply form's
// |t| + 0.5 lies within 1e-4 of an integer (exact = true takes the IEEE quotient instead)
__device__ __forceinline__ uint2 qpack_i8(const u32x4& v, float s, float rs, bool exact, bool& near) {
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const uint32_t ve = v[e >> 1];
    const float x = (e & 1) ? hi_bf(ve) : lo_bf(ve);
    const float t = exact ? x / s : x * rs;
    const float u = fabsf(t) + 0.5f, fr = u - truncf(u);
    near |= fr < 1e-4f || fr > 1.0f - 1e-4f;
    const int qi = (int)(t + (t >= 0.f ? 0.5f : -0.5f));
    w[e >> 2] |= ((uint32_t)qi & 0xffu) << (8 * (e & 3));
  }
  return make_uint2(w[0], w[1]);
}
// |x| maxima of bf16 pairs, two per register: with the sign bit cleared, bf16 bit patterns order as unsigned 16-bit
// integers the way their values do, so one AND and one packed 16-bit max (v_pk_max_u16) cover a pair of values.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 absmax2(u16x2 m, uint32_t p) {
  return __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, p & 0x7fff7fffu));
}
__device__ __forceinline__ float absmax_value(u16x2 m) { return __uint_as_float((uint32_t)max(m.x, m.y) << 16); }

// The exchange wave's side of a quantisation whose maximum it already holds (one float per lane: the LayerNorm's
// output h, in its registers): the wave-uniform scale and its reciprocal to qs[0], qs[1] for quant_pass_i8, written
// before the barrier that publishes the vector. Returns s. (Taking g's or a's maximum on the exchange wave while it
// gathers them was measured slower than the workgroup's own pass: 2263 / 2276 against 2285 tok/s.)
__device__ __forceinline__ float quant_scale_i8(float lane_amax, float* qs, int lane) {
  const float s = fmaxf(wave_max(lane_amax), 1e-5f) / 127.0f;
  if (lane == 0) {
    qs[0] = s;
    qs[1] = 1.0f / s;
  }
  return s;
}
// The quantising pass alone, by all the workgroup's waves after that barrier (every wave calls it at the same point;
// one barrier at the end): chunks of 8 values as quant_block_i8, scale from qs. Returns s.
template <int NCH>
__device__ __forceinline__ float quant_pass_i8(const uint32_t* src, uint32_t* dst, const float* qs, int tid) {
  const float s = qs[0], rs = qs[1];
#pragma unroll
  for (int c0 = 0; c0 < NCH; c0 += MK_T) {
    const int c = c0 + tid;
    if (c < NCH) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&src[4 * c]);
      bool near = false;
      uint2 q = qpack_i8(v, s, rs, false, near);
      if (__any(near)) {
        bool unused = false;
        q = qpack_i8(v, s, rs, true, unused);
      }
      *reinterpret_cast<uint2*>(&dst[2 * c]) = q;
    }
  }
  bar();
  return s;
}

// The quantisation of NCH chunks of 8 values (chunk c at src word 4 c, q to dst bytes 8 c .. 8 c + 7) by all the
// workgroup's waves (every wave calls it at the same point; it holds two barriers); returns s to every thread. One
// wave alone spent ~6 us on 8192 values (1.9 us on 2048), the workgroup ~0.6 us. red: one float per wave.
template <int NCH>
__device__ __forceinline__ float quant_block_i8(const uint32_t* src, uint32_t* dst, float* red, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  float amax = 0.f;
#pragma unroll
  for (int c0 = 0; c0 < NCH; c0 += MK_T) {
    const int c = c0 + tid;
    if (c < NCH) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&src[4 * c]);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t ve = v[e];
        amax = fmaxf(amax, fmaxf(fabsf(lo_bf(ve)), fabsf(hi_bf(ve))));
      }
    }
  }
  amax = wave_max(amax);
  if (lane == 0) red[wave] = amax;
  bar();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < MK_W + 1; w++) m = fmaxf(m, red[w]);
  const float s = fmaxf(m, 1e-5f) / 127.0f;
  const float rs = 1.0f / s;
#pragma unroll
  for (int c0 = 0; c0 < NCH; c0 += MK_T) {
    const int c = c0 + tid;
    if (c < NCH) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&src[4 * c]);
      bool near = false;
      uint2 q = qpack_i8(v, s, rs, false, near);
      if (__any(near)) {
        bool unused = false;
        q = qpack_i8(v, s, rs, true, unused);
      }
      *reinterpret_cast<uint2*>(&dst[2 * c]) = q;
    }
  }
  bar();
  return s;
}

__device__ __forceinline__ uint32_t amax_key32(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (u & 0xffff0000u) | (0xffffu - (uint32_t)idx);  // v is a bf16 value: its low 16 bits carry no order
}

// 16 bytes (two exchange words) at byte offset off of buf with an agent-scope load (sc1: past the non-coherent L2).
// Each 8-byte half is written by one single-copy-atomic store and carries its own epoch, so the two halves are
// checked separately. The compiler treats these loads as plain reads: a polling loop must pass a fresh (opaque) offset
// every pass, or the load is hoisted out of it and the loop never sees new data.
__device__ __forceinline__ u32x4 ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}

// The exchange wave's wait for words buf[0 .. NW) (NW a multiple of 128) with epoch ep, payloads into dst (LDS).
// Polls word 64 b + 63 of every block b (one load per lane, a few hundred bytes a round) until all carry ep, then
// reads every word in one batch (NW / 128 16-byte loads per lane, all in flight: one round trip), again where a word
// is still stale. (Re-reading whole buffers while waiting costs more than it saves: the polls of 224 workgroups share
// the memory pipeline with the weight stream.) FULL: no sentinel loop, the batch read is the poll, for a buffer that
// lands within about one round trip of the call (the attention output: its last head merges as the gather starts;
// two round trips instead of three, W8A8 decode 2287 -> 2326 tok/s; the g and x gathers wait longer and lose by it).
// fail: set on a timeout (with the error word); set on entry = return.
template <int NW, bool FULL = false>
__device__ void xgather(const uint64_t* __restrict__ buf, uint32_t ep, uint32_t* dst, uint32_t* err, bool& fail) {
  static_assert(NW % 128 == 0 && NW / 64 <= 64, "whole blocks, one sentinel per lane");
  constexpr int NB = NW / 64, NP = NW / 128;
  if (fail) return;
  const int lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(buf), (short)0, NW * 8, 0x00020000);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  auto timed_out = [&]() __attribute__((always_inline)) {
    if (__builtin_amdgcn_s_memrealtime() - t0 <= kTimeout) return false;
    fail = true;
    if (lane == 0) __hip_atomic_store(GLOBAL(uint32_t, err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  };
  for (; !FULL;) {  // sentinels: word 64 b + 63 of block b
    uint32_t so = (uint32_t)min(lane, NB - 1) * 512u + 508u;
    asm volatile("" : "+v"(so));  // a new offset each pass: the load is not hoisted out of the loop
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(r, so, 0, 16);
    if (!__any(hi != ep)) break;
    if (timed_out()) return;
    __builtin_amdgcn_s_sleep(2);
  }
  for (;;) {
    uint32_t lo = (uint32_t)lane * 16u;
    asm volatile("" : "+v"(lo));  // as above
    u32x4 v[NP];
#pragma unroll
    for (int j = 0; j < NP; j++) v[j] = ld_pair(r, lo + 1024u * j);
    int pending = 0;
#pragma unroll
    for (int j = 0; j < NP; j++) {
      const u32x4 t = v[j];
      pending |= (t[1] != ep) | (t[3] != ep);
    }
    if (!__any(pending)) {
#pragma unroll
      for (int j = 0; j < NP; j++) {
        const u32x4 t = v[j];
        *reinterpret_cast<uint2*>(&dst[2 * (lane + 64 * j)]) = make_uint2(t[0], t[2]);
      }
      return;
    }
    if (timed_out()) return;
  }
}

// f(integral_constant<int, I>) for I = 0 .. N - 1, unrolled at compile time (the slot index must be a constant: it
// selects registers and code paths)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef u32x4 Buf[8];  // one unit in flight: 2 rows x 4 chunks, a half fc2 row (8 chunks) or a proj row (4)

template <bool I8>
__global__ __launch_bounds__(MK_T) void decode_mk_kernel(MkArgs a) {
  using RC = RingCfg<I8>;
  constexpr int SA = RC::SA, B0 = RC::B0, B1 = RC::B1, BH = RC::BH, NSLOT = RC::NSLOT;
  __shared__ __attribute__((aligned(16))) uint32_t xs[MK_D / 2];  // x: the layer's input (bf16 pairs)
  // GEMV workgroups: g (fc1 output, 16 KB) then the attention output a (4 KB); attention workgroups: V rows (128 KB)
  __shared__ __attribute__((aligned(1024))) uint8_t big[MK_MAXKEYS * MK_HD * 2];
  __shared__ __attribute__((aligned(16))) uint16_t qkvh[3 * MK_HD];  // attention: the head's q, k, v (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t qr[MK_HD], kr[MK_HD];  // roped q, k (bf16)
  __shared__ float rec[MK_W][2 + MK_HD];
  __shared__ __attribute__((aligned(16))) uint32_t hs[MK_D / 2];  // GEMV workgroups: h = LN(x) (bf16 pairs)
  __shared__ float pb[4 * MK_RW], pc[MK_RW];  // fc2 quarter-row and proj partial sums
  __shared__ uint32_t sbest[MK_W];
  __shared__ uint64_t stab[MK_MAXL * MK_LP];
  __shared__ __attribute__((aligned(16))) uint32_t hq[MK_D / 4];  // W8A8: h quantised (int8)
  __shared__ float qred[MK_W + 1];                                // W8A8: per-wave maxima / a scale and reciprocal
  __shared__ int pbi[2 * MK_RW], pci[MK_RW];                      // W8A8: fc2 half-row and proj int32 sums
  uint32_t* gs = reinterpret_cast<uint32_t*>(big);
  uint32_t* as2 = gs + MK_F / 2;
  uint32_t* gq = reinterpret_cast<uint32_t*>(big + 65536);  // W8A8: g quantised (8 KB)
  uint32_t* aq = reinterpret_cast<uint32_t*>(big + 73728);  // W8A8: a quantised (2 KB)

  // wave-uniform by construction (readfirstlane): the compute / exchange split is a branch, not a predication that
  // would keep both sides' registers live at once
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), wg = blockIdx.x;
  const bool xw = wave == MK_XW;  // the exchange wave
  // The exchange wave issues first when it competes with the compute waves (its polls and publishes are what the
  // other workgroups wait for): ~5% per step.
  if (xw) __builtin_amdgcn_s_setprio(3);
  for (int i = tid; i < a.nl * MK_LP; i += MK_T) stab[i] = reinterpret_cast<const uint64_t*>(a.layers)[i];
  __syncthreads();
  const uint32_t base = a.ep[0];
  const int pos = min(max(a.state[1], 0), a.ctx - 1);  // the new token's position (its cached keys: rows 0 .. pos - 1)
  const int NL = a.nl;
  auto E = [&](int l, int p) __attribute__((always_inline)) { return base + 3u * (uint32_t)l + (uint32_t)p; };
  uint32_t* err = a.ep + 1;
  bool fail = false;  // exchange wave: a wait timed out

  // The exchange wave and the compute waves run separate loops that meet at the same barriers (5 per layer): one
  // loop with both roles as branches would be laid out as one straight region, both roles' registers live at once.
  int r0, nr;  // the workgroup's fc2 / proj rows
  row_group(wg, r0, nr);
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(xs);
  uint8_t* const pw = big + 24576;  // proj rows of the workgroup (4 KB each, 2 KB int8), after gs and as2
  constexpr uint32_t PROW = I8 ? MK_D : 2 * MK_D;  // bytes of a proj row
  if (wg >= MK_NG) {
    // ======================================================================= attention workgroup (one head)
    // The head's attention, then (V rows no longer needed in LDS) the workgroup's 8 fc2 / proj rows like a GEMV
    // workgroup's phases B and C.
    const int h = wg - MK_NG;
    if (xw) {
      // ---- exchange wave: q / k / v of the head, rope, output, append
      const int d = lane, jr = (d & 31) >> 1, d0 = d < 32 ? jr : d;
      const float cr = ldg(a.cs + (long)pos * 32 + 2 * jr), sr = ldg(a.cs + (long)pos * 32 + 2 * jr + 1);
      // x of the workgroup's rows (the residual): the step's input now, this workgroup's own output later
      if (lane < MK_RW / 2) xs[r0 / 2 + lane] = *GLOBAL(const uint32_t, a.x + r0 + 2 * lane);
      for (int l = 0; l < NL; l++) {
        const MkLayer L = layer_of(stab, l);
        uint64_t* ll = a.ll;  // opaque: the exchange addresses are rebuilt per layer, not hoisted
        asm volatile("" : "+s"(ll));
        const int ri = r0 + min(lane, nr - 1);
        const float b2v = ldg(L.b2 + ri), bpv = ldg(L.bp + ri);
        const float sw2v = I8 ? ldg(L.sw2 + ri) : 0.f, swpv = I8 ? ldg(L.swp + ri) : 0.f;
        // 96 words: q at h * 32, k at 1024 + h * 32, v at 2048 + h * 32
        if (!fail) {
          const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
          const int w1 = (lane >> 5) * 1024 + h * 32 + (lane & 31), w2 = 2048 + h * 32 + (lane & 31);
          for (;;) {
            const uint64_t v1 = ld_word(ll + LL_QKV + w1), v2 = ld_word(ll + LL_QKV + w2);
            const bool ok = (uint32_t)(v1 >> 32) == E(l, 1) && (lane >= 32 || (uint32_t)(v2 >> 32) == E(l, 1));
            if (!__any(!ok)) {
              reinterpret_cast<uint32_t*>(qkvh)[lane] = (uint32_t)v1;
              if (lane < 32) reinterpret_cast<uint32_t*>(qkvh)[64 + lane] = (uint32_t)v2;
              break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kTimeout) {
              fail = true;
              if (lane == 0) __hip_atomic_store(GLOBAL(uint32_t, err), 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
          }
        }
        // rope of the new token's q and k (fp32, rope.hip's arithmetic): output dim d < 32 pairs input dims
        // (d >> 1, 16 + (d >> 1)); the roped k and the raw v are appended at pos at the end of the layer
        const float qa = bf2f(qkvh[d0]), qb = bf2f(qkvh[16 + jr]);
        const float ka = bf2f(qkvh[MK_HD + d0]), kb = bf2f(qkvh[MK_HD + 16 + jr]);
        const float qo = __fadd_rn(__fmul_rn(qa, sr), __fmul_rn(qb, cr)), qe = __fsub_rn(__fmul_rn(qa, cr), __fmul_rn(qb, sr));
        const float ko = __fadd_rn(__fmul_rn(ka, sr), __fmul_rn(kb, cr)), ke = __fsub_rn(__fmul_rn(ka, cr), __fmul_rn(kb, sr));
        const float qv = d < 32 ? ((d & 1) ? qo : qe) : qa;
        const float kv = d < 32 ? ((d & 1) ? ko : ke) : ka;
        qr[d] = f2bf(qv);
        const uint16_t kapp = f2bf(kv);
        kr[d] = kapp;
        const uint16_t vapp = qkvh[2 * MK_HD + d];
        bar();  // q, k, v ready
        bar();  // the 8 waves' (m, l, o) in rec
        if (lane < MK_HD / 2) {  // two output dims per lane -> one word
          float M = -INFINITY;
#pragma unroll
          for (int w = 0; w < MK_W; w++) M = fmaxf(M, rec[w][0]);
          float Lt = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
          for (int w = 0; w < MK_W; w++) {
            const float f = __builtin_amdgcn_exp2f(rec[w][0] - M);
            Lt += rec[w][1] * f;
            a0 += rec[w][2 + 2 * lane] * f;
            a1 += rec[w][3 + 2 * lane] * f;
          }
          st_word(ll + LL_A + h * 32 + lane, E(l, 2), pack2(a0 / Lt, a1 / Lt));
        }
        // the append (read by later steps only)
        *GLOBAL(uint16_t, L.kc + ((long)h * a.ctx + pos) * MK_HD + lane) = kapp;
        *GLOBAL(uint16_t, L.vc + ((long)h * a.ctx + pos) * MK_HD + lane) = vapp;
        // rec / qkvh / qr / kr are rewritten only after the next layer's first barrier
        // ---- the workgroup's fc2 / proj rows (gs, as2 over the V rows: the compute waves are past them)
        xgather<MK_F / 4>(ll + LL_G, E(l, 1), gs, err, fail);
        if (!I8) bar();  // g1 ready
        xgather<MK_F / 4>(ll + LL_G + MK_F / 4, E(l, 1), gs + MK_F / 4, err, fail);
        float sg = 0.f, sa = 0.f;
        bar();  // g2 ready (W8A8: g gathered, then quantised by all waves)
        if (I8) sg = quant_block_i8<MK_F / 8>(gs, gq, qred, tid);
        xgather<MK_D / 2, true>(ll + LL_A, E(l, 2), as2, err, fail);
        bar();  // a ready (W8A8: then quantised by all waves; the compute waves are done with phase B)
        if (I8) sa = quant_block_i8<MK_D / 8>(as2, aq, qred, tid);
        bar();  // the partial sums in pb / pc
        float xn = 0.f;
        if (lane < nr) {
          if (I8) {
            const float y2 = rbf(((float)(pbi[2 * lane] + pbi[2 * lane + 1]) * sg) * sw2v + b2v);
            xn = rbf(y2 + rbf(rbf(((float)pci[lane] * sa) * swpv + bpv) + bf2f(xb[r0 + lane])));
          } else {
            const float y2 = rbf(((pb[4 * lane] + pb[4 * lane + 1]) + (pb[4 * lane + 2] + pb[4 * lane + 3])) + b2v);
            xn = rbf(y2 + rbf(rbf(pc[lane] + bpv) + bf2f(xb[r0 + lane])));
          }
        }
        const float xn1 = __shfl_down(xn, 1, 64);
        if (lane < nr && !(lane & 1)) {
          const uint32_t w = pack2(xn, xn1);
          st_word(ll + LL_X + (r0 + lane) / 2, E(l, 3), w);
          xs[(r0 + lane) / 2] = w;  // the next layer's residual
        }
      }
    } else {
      // ---- compute waves: the cached keys 0 .. pos - 1 of the head, K rows into registers and V rows into LDS (row
      // key at byte 128 key), issued before the exchange wave's wait for q / k / v; lane l of wave w takes key
      // w * 8 + (l >> 3) + 64 r in round r, dims 8 (l & 7) .. + 7. The buffer range of both caches ends at row pos, so
      // rows at and past pos read as zeros (masked below; the new token's own key is scored by wave 0 from LDS).
      // One-pass softmax per wave, merged by the exchange wave.
      const int sub = lane & 7, kg = lane >> 3;
      const uint32_t koff = (uint32_t)(wave * 8 + kg) * 128u + (uint32_t)sub * 16u;
      for (int l = 0; l < NL; l++) {
        const MkLayer L = layer_of(stab, l);
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(L.kc + (long)h * a.ctx * MK_HD, (short)0, pos * 128, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(L.vc + (long)h * a.ctx * MK_HD, (short)0, pos * 128, 0x00020000);
        uint32_t ko = koff;
        asm volatile("" : "+v"(ko));
        u32x4 kk[MK_ROUNDS];
#pragma unroll
        for (int r = 0; r < MK_ROUNDS; r++) {
          kk[r] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 8192u * r, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rv, (__attribute__((address_space(3))) void*)(big + (wave * 8 + 64 * r) * 128), 16, ko + 8192u * r, 0, 0, 0);
        }
        bar();  // q, k, v ready
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's K registers and V rows have landed
        const u32x4 qp = *reinterpret_cast<const u32x4*>(&qr[sub * 8]);
        float sv[MK_ROUNDS];
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < MK_ROUNDS; r++) {
          const int key = wave * 8 + kg + 64 * r;
          float sc = dot8d(kk[r], qp, 0.f);
          sc += __shfl_xor(sc, 1, 64);
          sc += __shfl_xor(sc, 2, 64);
          sc += __shfl_xor(sc, 4, 64);
          sc = key < pos ? sc * a.scale_log2 : -INFINITY;
          sv[r] = sc;
          mb = fmaxf(mb, sc);
        }
        float snew = -INFINITY;  // the new token's key, wave 0
        if (wave == 0) {
          float sc = dot8d(*reinterpret_cast<const u32x4*>(&kr[sub * 8]), qp, 0.f);
          sc += __shfl_xor(sc, 1, 64);
          sc += __shfl_xor(sc, 2, 64);
          sc += __shfl_xor(sc, 4, 64);
          snew = sc * a.scale_log2;
          mb = fmaxf(mb, snew);
        }
        const float m = fmaxf(wave_max(mb), -1e30f);  // a wave with no key in range: p = 0, not NaN
        float lsum = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < MK_ROUNDS; r++) {
          // rows past the range: p = 0, and the LDS row is zeroed here whatever the copy left in it (0 x NaN = NaN)
          const u32x4 zero4 = {0u, 0u, 0u, 0u};
          const u32x4 vl = *reinterpret_cast<const u32x4*>(big + (wave * 8 + kg + 64 * r) * 128 + sub * 16);
          const u32x4 vv = wave * 8 + kg + 64 * r < pos ? vl : zero4;
          const float pr = rbf(__builtin_amdgcn_exp2f(sv[r] - m));
          if (sub == 0) lsum += pr;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t ve = vv[e];
            o[2 * e] = __builtin_fmaf(pr, lo_bf(ve), o[2 * e]);
            o[2 * e + 1] = __builtin_fmaf(pr, hi_bf(ve), o[2 * e + 1]);
          }
        }
        if (wave == 0 && kg == 0) {
          const u32x4 vv = *reinterpret_cast<const u32x4*>(&qkvh[2 * MK_HD + sub * 8]);
          const float pr = rbf(__builtin_amdgcn_exp2f(snew - m));
          if (sub == 0) lsum += pr;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t ve = vv[e];
            o[2 * e] = __builtin_fmaf(pr, lo_bf(ve), o[2 * e]);
            o[2 * e + 1] = __builtin_fmaf(pr, hi_bf(ve), o[2 * e + 1]);
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
        bar();  // the 8 waves' (m, l, o) in rec; every V row read
        // ---- the workgroup's fc2 / proj rows: this wave's row r0 + wave of fc2 into registers (4 KB units: quarters,
        // or int8 halves), its proj row into LDS (over the V rows, read by now)
        uint32_t lo = (uint32_t)lane * 16u;
        asm volatile("" : "+v"(lo));
        constexpr int NU = I8 ? 2 : JBA;
        u32x4 wb[NU][4];
#pragma unroll
        for (int j = 0; j < NU; j++) {
          const uint32_t o = (uint32_t)(r0 + wave) * (I8 ? MK_F : MK_F * 2u) + (uint32_t)j * 4096u + lo;
#pragma unroll
          for (int i = 0; i < 4; i++) wb[j][i] = ldw(L.w2, o + 1024u * i);
        }
#pragma unroll
        for (int j = 0; j < JCA; j++) {
          const int u = wave + MK_W * j;
#pragma unroll
          for (int i = 0; i < (int)PROW / 1024; i++)
            dma16s(L.wp, (uint32_t)(r0 + u) * PROW + 1024u * i + lo, lds_off(pw) + (uint32_t)u * PROW + 1024u * i);
        }
        if constexpr (I8) {
          bar();  // g gathered
          quant_block_i8<MK_F / 8>(gs, gq, qred, tid);
#pragma unroll
          for (int j = 0; j < NU; j++) {  // half j of the row
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc = dot16_i8(*reinterpret_cast<const u32x4*>(&gq[j * 1024 + 4 * (lane + 64 * i)]), wb[j][i], acc);
            const int t = wave_total_i(acc);
            if (lane == 0) pbi[2 * wave + j] = t;
          }
        } else {
#pragma unroll
          for (int j = 0; j < NU; j++) {
            if (j == 0) bar();  // g1 ready
            if (j == 2) bar();  // g2 ready
            const uint32_t* gh = gs + j * (MK_D / 2);
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc = dot8d(wb[j][i], *reinterpret_cast<const u32x4*>(&gh[(lane + 64 * i) * 4]), acc);
            const float t = wave_total(acc);
            if (lane == 0) pb[4 * wave + j] = t;
          }
        }
        bar();  // a ready
        if constexpr (I8) quant_block_i8<MK_D / 8>(as2, aq, qred, tid);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the proj rows have landed
#pragma unroll
        for (int j = 0; j < JCA; j++) {
          const int u = wave + MK_W * j;
          const uint8_t* pr = pw + u * PROW;
          if constexpr (I8) {
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 2; i++)
              acc = dot16_i8(*reinterpret_cast<const u32x4*>(&aq[4 * (lane + 64 * i)]),
                             *reinterpret_cast<const u32x4*>(pr + (lane + 64 * i) * 16), acc);
            const int t = wave_total_i(acc);
            if (lane == 0) pci[u] = t;
          } else {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc = dot8d(*reinterpret_cast<const u32x4*>(pr + (lane + 64 * i) * 16),
                          *reinterpret_cast<const u32x4*>(&as2[(lane + 64 * i) * 4]), acc);
            const float t = wave_total(acc);
            if (lane == 0) pc[u] = t;
          }
        }
        bar();  // the partial sums in pb / pc; every read of gs, as2, pw done (the next layer's V rows may land)
      }
    }
  } else {
    // ======================================================================= GEMV workgroup
    if (xw) {
      // ---- exchange wave: x in, h = LN(x) for the compute waves, g and a in, this workgroup's x' rows out
      for (int l = 0; l < NL; l++) {
        const MkLayer L = layer_of(stab, l);
        uint64_t* ll = a.ll;  // opaque: the exchange addresses are rebuilt per layer, not hoisted
        asm volatile("" : "+s"(ll));
        // the LayerNorm parameters and the workgroup's fc2 / proj biases (row r0 + lane), loaded while x is awaited
        u32x4 xc[4], gc[4], bc[4];
        load_vec_g<4>(gc, L.ln_g, lane);
        load_vec_g<4>(bc, L.ln_b, lane);
        const int ri = r0 + min(lane, nr - 1);
        const float b2v = ldg(L.b2 + ri), bpv = ldg(L.bp + ri);
        const float sw2v = I8 ? ldg(L.sw2 + ri) : 0.f, swpv = I8 ? ldg(L.swp + ri) : 0.f;
        if (l == 0) {
          load_vec_g<4>(xc, a.x, lane);
#pragma unroll
          for (int i = 0; i < 4; i++) reinterpret_cast<u32x4*>(xs)[lane + 64 * i] = xc[i];
        } else {
          xgather<MK_D / 2>(ll + LL_X, E(l - 1, 3), xs, err, fail);
          load_vec<4>(xc, xb, lane);
        }
        ln_chunks<4, true>(xc, gc, bc, a.eps, MK_D, lane);
        u16x2 hm = {0, 0};  // W8A8: this lane's |h| maximum, for the scale
#pragma unroll
        for (int i = 0; i < 4; i++) {
          reinterpret_cast<u32x4*>(hs)[lane + 64 * i] = xc[i];
          if (I8) {
#pragma unroll
            for (int e = 0; e < 4; e++) hm = absmax2(hm, xc[i][e]);
          }
        }
        if (I8) quant_scale_i8(absmax_value(hm), qred, lane);
        bar();  // h ready (W8A8: with its scale; then quantised by all waves, shared by qkv and fc1, md2fast.py:174)
        if (I8) quant_pass_i8<MK_D / 8>(hs, hq, qred, tid);
        bar();  // the workgroup's phase A done
        xgather<MK_F / 4>(ll + LL_G, E(l, 1), gs, err, fail);
        if (!I8) bar();  // g1 ready
        xgather<MK_F / 4>(ll + LL_G + MK_F / 4, E(l, 1), gs + MK_F / 4, err, fail);
        float sg = 0.f, sa = 0.f;
        bar();  // g2 ready (W8A8: g gathered, then quantised by all waves)
        if (I8) sg = quant_block_i8<MK_F / 8>(gs, gq, qred, tid);
        xgather<MK_D / 2, true>(ll + LL_A, E(l, 2), as2, err, fail);
        bar();  // a ready (W8A8: then quantised by all waves; the compute waves are done with phase B)
        if (I8) sa = quant_block_i8<MK_D / 8>(as2, aq, qred, tid);
        bar();  // the partial sums in pb / pc
        // x'[n] = bf16(y2[n] + bf16(bf16(a Wp^T + bp)[n] + x[n])), y2 = bf16(g W2^T + b2): row r0 + lane (W8A8: each
        // Linear's fp32 dequant ((acc s_act) s_w) + b rounded once, i8gemm.hip:181-197)
        float xn = 0.f;
        if (lane < nr) {
          if (I8) {
            const float y2 = rbf(((float)(pbi[2 * lane] + pbi[2 * lane + 1]) * sg) * sw2v + b2v);
            xn = rbf(y2 + rbf(rbf(((float)pci[lane] * sa) * swpv + bpv) + bf2f(xb[r0 + lane])));
          } else {
            const float y2 = rbf(((pb[4 * lane] + pb[4 * lane + 1]) + (pb[4 * lane + 2] + pb[4 * lane + 3])) + b2v);
            xn = rbf(y2 + rbf(rbf(pc[lane] + bpv) + bf2f(xb[r0 + lane])));
          }
        }
        const float xn1 = __shfl_down(xn, 1, 64);
        if (lane < nr && !(lane & 1)) st_word(ll + LL_X + (r0 + lane) / 2, E(l, 3), pack2(xn, xn1));
      }
    } else if (wave < GW) {
      // ---- GEMV waves: a ring of NBUF 4 KB weight units, slot s of a layer in buffer s % NBUF, the unit NBUF slots
      // ahead issued as soon as a slot is reduced (across phase and layer boundaries):
      //   slots [0, SA): phase A, the pair rot_wave(wg, wave, k) + k MK_NGW (k = s / 2) of [Wqkv | Wfc1] rows (qkv
      //   pairs first), row s % 2
      //   slots [B0, B1): phase B, unit u = wave + GW (s - B0) < 4 nr: quarter u % 4 of fc2 row r0 + u / 4
      // and phase C from LDS: proj row r0 + u (u = wave + GW j < nr) at pw + 4 KB u
      u32x4 buf[NBUF][4];
      float bqr[NBUF], bqr2[NBUF], sqr[NBUF], sqr2[NBUF];  // phase A: the unit's biases (W8A8: both rows', and scales)
      const uint32_t pwo = lds_off(pw);
      // real = false (the next-layer slots of the last layer): the same loads from the LayerNorm gamma, discarded
      auto issue = [&](auto sc, const MkLayer& L, uint32_t lo, bool real) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        u32x4(&b)[4] = buf[s % NBUF];
        if constexpr (I8 && s < SA) {  // the row pair of round s: 2 x 2 KB, rows 2 p, 2 p + 1
          const int p = rot_wave(wg, wave, s) + s * MK_NGW;
          const uint32_t o = real ? (uint32_t)p * (MK_D * 2u) + lo : lo;
#pragma unroll
          for (int i = 0; i < 4; i++) b[i] = ldw(real ? L.wqf : L.ln_g, o + 1024u * i);
          bqr[s % NBUF] = ldg(L.bqf + 2 * p);
          bqr2[s % NBUF] = ldg(L.bqf + 2 * p + 1);
          sqr[s % NBUF] = ldg(L.sqf + 2 * p);
          sqr2[s % NBUF] = ldg(L.sqf + 2 * p + 1);
        } else if constexpr (I8 && s >= B0 && s < B1) {  // half u & 1 of int8 fc2 row r0 + u / 2
          const int u = wave + GW * (s - B0);
          const uint32_t o = (uint32_t)(r0 + (u >> 1)) * (uint32_t)MK_F + (uint32_t)(u & 1) * 4096u + lo;
#pragma unroll
          for (int i = 0; i < 4; i++) b[i] = ldw(L.w2, o + 1024u * i);
        } else if constexpr (s < SA) {
          const int row = 2 * (rot_wave(wg, wave, s >> 1) + (s >> 1) * MK_NGW) + (s & 1);
          const uint32_t o = real ? (uint32_t)row * (MK_D * 2u) + lo : lo;
#pragma unroll
          for (int i = 0; i < 4; i++) b[i] = ldw(real ? L.wqf : L.ln_g, o + 1024u * i);
          bqr[s % NBUF] = ldg(L.bqf + row);
        } else if constexpr (s >= B0 && s < B1) {
          // a slot past the workgroup's units reads the LayerNorm gamma (4 KB, in cache) instead: every slot issues
          // the same loads, so the compiler's wait counts stay exact (a conditional load makes them drain everything)
          const int rw = b_row(wave, s - B0), q = b_quarter(s - B0);
          const bool ok = rw < nr;
          const uint32_t o = ok ? (uint32_t)(r0 + rw) * (MK_F * 2u) + (uint32_t)q * (MK_D * 2u) + lo : lo;
#pragma unroll
          for (int i = 0; i < 4; i++) b[i] = ldw(ok ? L.w2 : L.ln_g, o + 1024u * i);
        }
      };
      u32x4 hc[4];
      float accE = 0.f, bE = 0.f;  // phase A: the even row of the current pair
      // The pair words are published in three bursts, one vector store each: after the last round that holds qkv
      // pairs, after the last one with pairs of g[0, 4096), and at the end of phase A. A store holds back this wave's
      // later waits until it completes (the counter completes in order), ~2 us at agent scope under load: one per pair
      // would stall the weight stream KA times.
      uint32_t wq[KA];
      u32x4 hqv[2];  // W8A8: this lane's chunks (16 int8 each) of the quantised h
      float sh = 0.f;
      // the burst that ends with pair round k (lane i publishes the word of round k0 + i)
      auto burst = [&](auto kc, uint64_t* ll, uint32_t ep) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        if constexpr (k == KQ || k == KG1 || k == KA - 1) {
          constexpr int k0 = k == KQ ? 0 : k == KG1 ? KQ + 1 : KG1 + 1;
          uint32_t w = wq[k0];
#pragma unroll
          for (int j = k0 + 1; j <= k; j++) w = lane == j - k0 ? wq[j] : w;
          const int kl = k0 + lane;
          if (lane <= k - k0) st_word(ll + LL_QKV + rot_wave(wg, wave, kl) + kl * MK_NGW, ep, w);
        }
      };
      auto compute = [&](auto sc, uint64_t* ll, uint32_t ep) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        const u32x4(&b)[4] = buf[s % NBUF];
        if constexpr (I8 && s < SA) {  // the pair: exact int32 sums, dequant ((acc s_h) s_w) + b, GELU on fc1 rows
          const int p = rot_wave(wg, wave, s) + s * MK_NGW;
          int a0 = dot16_i8(hqv[0], b[0], 0), a1 = dot16_i8(hqv[0], b[2], 0);
          a0 = dot16_i8(hqv[1], b[1], a0);
          a1 = dot16_i8(hqv[1], b[3], a1);
          float ve = ((float)wave_total_i(a0) * sh) * sqr[s % NBUF] + bqr[s % NBUF];
          float vo = ((float)wave_total_i(a1) * sh) * sqr2[s % NBUF] + bqr2[s % NBUF];
          if (2 * p >= MK_NQKV) {
            ve = gelu_tanh(ve);
            vo = gelu_tanh(vo);
          }
          wq[s] = pack2(ve, vo);
          burst(std::integral_constant<int, s>{}, ll, ep);
        } else if constexpr (I8 && s >= B0 && s < B1) {
          const int u = wave + GW * (s - B0);
          int acc = 0;
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc = dot16_i8(*reinterpret_cast<const u32x4*>(&gq[(u & 1) * 1024 + 4 * (lane + 64 * i)]), b[i], acc);
          const int t = wave_total_i(acc);
          if (lane == 0) pbi[u] = t;  // row u / 2, half u & 1
        } else if constexpr (s < SA) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 4; i++) acc = dot8d(b[i], hc[i], acc);
          if constexpr (!(s & 1)) {
            accE = acc;
            bE = bqr[s % NBUF];
          } else {  // the pair: + bias, GELU on fc1 rows, one exchange word (qkv and g words are contiguous)
            constexpr int k = s >> 1;
            const int pr = rot_wave(wg, wave, k) + k * MK_NGW;
            float ve = rbf(wave_total(accE) + bE), vo = rbf(wave_total(acc) + bqr[s % NBUF]);
            if (2 * pr >= MK_NQKV) {
              ve = rbf(gelu_tanh(ve));
              vo = rbf(gelu_tanh(vo));
            }
            wq[k] = pack2(ve, vo);
            burst(std::integral_constant<int, k>{}, ll, ep);
          }
        } else if constexpr (s >= B0 && s < B1) {
          const int rw = b_row(wave, s - B0), q = b_quarter(s - B0);
          if (rw < nr) {
            const uint32_t* gq = gs + q * (MK_D / 2);
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc = dot8d(b[i], *reinterpret_cast<const u32x4*>(&gq[(lane + 64 * i) * 4]), acc);
            const float t = wave_total(acc);
            if (lane == 0) pb[4 * rw + q] = t;
          }
        }
      };
      {
        const MkLayer L0 = layer_of(stab, 0);
        uint32_t lo = (uint32_t)lane * 16u;
        asm volatile("" : "+v"(lo));
        static_for<PF>([&](auto sc) __attribute__((always_inline)) { issue(sc, L0, lo, true); });
      }
      for (int l = 0; l < NL; l++) {
        const MkLayer L = layer_of(stab, l);
        const bool more = l + 1 < NL;
        const MkLayer Ln = layer_of(stab, more ? l + 1 : l);
        // the lane's byte offset and the exchange base, opaque to the compiler: the addresses derived from them are
        // rebuilt every layer instead of being hoisted out of the loop (live across it, they spill)
        uint32_t lo = (uint32_t)lane * 16u;
        asm volatile("" : "+v"(lo));
        uint64_t* ll = a.ll;
        asm volatile("" : "+s"(ll));
        // this wave's proj rows into LDS (DMA), landed before the h barrier: the wait costs nothing there (x comes
        // later), and none is needed later, when the next layer's first units are in flight
#pragma unroll
        for (int j = 0; j < JC; j++) {
          const int u = wave + GW * j;
          if (u < nr) {
#pragma unroll
            for (int i = 0; i < (int)PROW / 1024; i++)
              dma16s(L.wp, (uint32_t)(r0 + u) * PROW + 1024u * i + lo, pwo + (uint32_t)u * PROW + 1024u * i);
          }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bar();  // h ready
        static_for<(DIST > PF ? DIST - PF : 0)>([&](auto sc) __attribute__((always_inline)) {
          issue(std::integral_constant<int, PF + decltype(sc)::value>{}, L, lo, true);
        });
        if constexpr (I8) {
          sh = quant_pass_i8<MK_D / 8>(hs, hq, qred, tid);
          hqv[0] = *reinterpret_cast<const u32x4*>(&hq[4 * lane]);
          hqv[1] = *reinterpret_cast<const u32x4*>(&hq[4 * (lane + 64)]);
        } else {
          load_vec<4>(hc, reinterpret_cast<const uint16_t*>(hs), lane);
        }
        static_for<NSLOT>([&](auto sc) __attribute__((always_inline)) {
          constexpr int s = decltype(sc)::value;
          if constexpr (s == B0) {
            bar();  // phase A done
            bar();  // g1 ready (W8A8: all of g gathered)
            if constexpr (I8) quant_block_i8<MK_F / 8>(gs, gq, qred, tid);
          }
          if constexpr (!I8 && s == BH) bar();  // g2 ready
          compute(sc, ll, E(l, 1));
          // the freed buffer's next unit (sched_barrier: kept after the reduction that frees it; the scheduler would
          // otherwise hoist the loads and need more buffers)
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (s + DIST < NSLOT) {
            if constexpr (s + DIST >= PF) issue(std::integral_constant<int, s + DIST>{}, L, lo, true);
          } else if constexpr (s + DIST - NSLOT < PF) {
            issue(std::integral_constant<int, s + DIST - NSLOT>{}, Ln, lo, more);
          }
          __builtin_amdgcn_sched_barrier(0);
        });
        // the next layer's units DIST .. PF - 1 (their buffers are free now)
        static_for<(PF > DIST ? PF - DIST : 0)>([&](auto sc) __attribute__((always_inline)) {
          issue(std::integral_constant<int, DIST + decltype(sc)::value>{}, Ln, lo, more);
        });
        bar();  // a ready
        if constexpr (I8) quant_block_i8<MK_D / 8>(as2, aq, qred, tid);
        // ---- phase C from LDS
#pragma unroll
        for (int j = 0; j < JC; j++) {
          const int u = wave + GW * j;
          if (u < nr) {
            const uint8_t* pr = pw + u * PROW;
            if constexpr (I8) {
              int acc = 0;
#pragma unroll
              for (int i = 0; i < 2; i++)
                acc = dot16_i8(*reinterpret_cast<const u32x4*>(&aq[4 * (lane + 64 * i)]),
                               *reinterpret_cast<const u32x4*>(pr + (lane + 64 * i) * 16), acc);
              const int t = wave_total_i(acc);
              if (lane == 0) pci[u] = t;
            } else {
              float acc = 0.f;
#pragma unroll
              for (int i = 0; i < 4; i++)
                acc = dot8d(*reinterpret_cast<const u32x4*>(pr + (lane + 64 * i) * 16),
                            *reinterpret_cast<const u32x4*>(&as2[(lane + 64 * i) * 4]), acc);
              const float t = wave_total(acc);
              if (lane == 0) pc[u] = t;
            }
          }
        }
        bar();  // the partial sums in pb / pc; every read of hs, gs, as2, pw done
      }
    } else {
      for (int l = 0; l < NL; l++)  // waves past GW: the same barriers per layer
        for (int i = 0; i < NBAR; i++) bar();
    }
  }

  // ========================================================================= LM head + argmax (all workgroups)
  {
    // 2048 compute waves; job round i: 2-row job jidx(i) = SJ i + (this wave's index, rotated over each group of 8
    // workgroups as in phase A)
    constexpr int SJ = MK_G * MK_W;
    auto jidx = [&](int i) __attribute__((always_inline)) {
      return SJ * i + ((wg & ~7) + ((wg + (MK_ROT ? i : 0)) & 7)) * MK_W + wave;
    };
    const int njobs = (a.V + 1) / 2;
    uint32_t lo = (uint32_t)lane * 16u;
    asm volatile("" : "+v"(lo));
    uint64_t* ll = a.ll;
    asm volatile("" : "+s"(ll));
    Buf w0, w1;
    float bj0 = 0.f, bj1 = 0.f;
    auto issue = [&](Buf& b, float& bj, int j) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const uint32_t o = (uint32_t)min(2 * j + r, a.V - 1) * (MK_D * 2u) + lo;
#pragma unroll
        for (int i = 0; i < 4; i++) b[4 * r + i] = ldw(a.wlm, o + 1024u * i);
      }
      bj = ldg(a.blm + min(2 * j + (lane >> 5), a.V - 1));
    };
    uint32_t best = 0u;
    u32x4 xc[4];
    auto job = [&](const Buf& b, float bj, int j) __attribute__((always_inline)) {
      float acc[2];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        acc[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r] = dot8d(b[4 * r + i], xc[i], acc[r]);
      }
      const int n = 2 * j + (lane >> 5);
      const float t0 = wave_total(acc[0]), t1 = wave_total(acc[1]);
      const float tot = lane < 32 ? t0 : t1;
      if (n < a.V) {
        const float v = rbf(tot + bj);
        if (a.logits && (lane & 31) == 0) *GLOBAL(uint16_t, a.logits + n) = f2bf(v);
        const uint32_t k = amax_key32(v, n);
        best = k > best ? k : best;
      }
    };
    u32x4 gc[4], bc[4];
    if (!xw) {
      if (jidx(0) < njobs) issue(w0, bj0, jidx(0));
      if (jidx(1) < njobs) issue(w1, bj1, jidx(1));
      load_vec_g<4>(gc, a.lnf_g, lane);
      load_vec_g<4>(bc, a.lnf_b, lane);
    } else {
      xgather<MK_D / 2>(ll + LL_X, E(NL - 1, 3), xs, err, fail);
    }
    bar();  // x ready
    if (!xw) {
      load_vec<4>(xc, reinterpret_cast<const uint16_t*>(xs), lane);
      ln_chunks<4, true>(xc, gc, bc, a.eps, MK_D, lane);
      for (int i = 0; jidx(i) < njobs; i += 2) {
        job(w0, bj0, jidx(i));
        __builtin_amdgcn_sched_barrier(0);
        if (jidx(i + 2) < njobs) issue(w0, bj0, jidx(i + 2));
        if (jidx(i + 1) < njobs) {
          job(w1, bj1, jidx(i + 1));
          __builtin_amdgcn_sched_barrier(0);
          if (jidx(i + 3) < njobs) issue(w1, bj1, jidx(i + 3));
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t t = __shfl_xor(best, o, 64);
        best = t > best ? t : best;
      }
      if (lane == 0) sbest[wave] = best;
    }
    bar();
    if (xw && lane == 0) {
      uint32_t b = sbest[0];
#pragma unroll
      for (int w = 1; w < MK_W; w++) b = sbest[w] > b ? sbest[w] : b;
      st_word(ll + LL_AM + wg, base + 3u * (uint32_t)NL + 1u, b);
    }
  }
  if (wg != 0 || !xw) return;
  // ---- workgroup 0's exchange wave: the token, the bookkeeping of embed_step_kernel, the next embedding, the next
  // epoch base (every workgroup has read the old ones: their argmax words come after)
  xgather<MK_G>(a.ll + LL_AM, base + 3u * (uint32_t)NL + 1u, xs, err, fail);
  uint32_t b = 0u;
#pragma unroll
  for (int i = 0; i < MK_G / 64; i++) b = xs[lane + 64 * i] > b ? xs[lane + 64 * i] : b;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t t = __shfl_xor(b, o, 64);
    b = t > b ? t : b;
  }
  const int tok = min((int)(0xffffu - (b & 0xffffu)), a.V - 1);
  if (lane == 0) {
    const int s = a.state[0];
    if (s < a.cap) {
      a.tokens[s] = tok;
      a.state[1] = a.pos_base + s;
      a.state[0] = s + 1;
    }
    if (!fail) a.ep[0] = base + 3u * (uint32_t)NL + 2u;
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
    *GLOBAL(u32x4, a.x + (lane + 64 * i) * 8) = ldg_vec(a.wte + (long)tok * MK_D + (lane + 64 * i) * 8);
}

}  // namespace

extern "C" int mx_decode_mk_words(void) { return LL_WORDS; }

extern "C" int mx_decode_mk_grid(void) { return MK_G; }

namespace {
template <bool I8>
int launch_mk(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g, const uint16_t* lnf_b,
              const uint16_t* wlm, const float* blm, int V, const uint16_t* wte, const float* cs, float eps, float scale,
              uint16_t* x, int* state, int pos_base, int* tokens, int cap, uint16_t* logits, uint64_t* ll,
              uint32_t* ep) {
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
  hipLaunchKernelGGL(decode_mk_kernel<I8>, dim3(MK_G), dim3(MK_T), 0, st, a);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
}  // namespace

// One greedy decode step of the 2048-wide, 32-head text model in one launch (decode_mk_kernel): layers[nl] describes
// every layer's weights and cache (device memory), x the step's input embedding (replaced by the next step's), state /
// tokens / cap / pos_base as mx_embed_step; logits optional (V bf16). ll: mx_decode_mk_words() zeroed words, ep: 2
// words {epoch base, error} zeroed once, both owned by one decoder (the kernel advances the base). Needs
// mx_decode_mk_grid() CUs (one workgroup on each, all resident) and ctx <= 1024 (the keys one pass holds).
extern "C" int mx_decode_step_mk(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g,
                                 const uint16_t* lnf_b, const uint16_t* wlm, const float* blm, int V,
                                 const uint16_t* wte, const float* cs, float eps, float scale, uint16_t* x, int* state,
                                 int pos_base, int* tokens, int cap, uint16_t* logits, uint64_t* ll, uint32_t* ep) {
  return launch_mk<false>(st, layers, nl, ctx, lnf_g, lnf_b, wlm, blm, V, wte, cs, eps, scale, x, state, pos_base,
                          tokens, cap, logits, ll, ep);
}

// The same step with the W8A8 text Linears: each descriptor's wqf / w2 / wp are int8 (the same shapes, one byte per
// weight) and its sqf / sw2 / swp hold their fp32 per-row scales; the LM head stays bf16.
extern "C" int mx_decode_step_mk_i8(hipStream_t st, const void* layers, int nl, int ctx, const uint16_t* lnf_g,
                                    const uint16_t* lnf_b, const uint16_t* wlm, const float* blm, int V,
                                    const uint16_t* wte, const float* cs, float eps, float scale, uint16_t* x,
                                    int* state, int pos_base, int* tokens, int cap, uint16_t* logits, uint64_t* ll,
                                    uint32_t* ep) {
  return launch_mk<true>(st, layers, nl, ctx, lnf_g, lnf_b, wlm, blm, V, wte, cs, eps, scale, x, state, pos_base,
                         tokens, cap, logits, ll, ep);
}

// Bytes of one layer descriptor in the layers array of mx_decode_step_mk(_i8): 13 device pointers (ln_g, ln_b, wqf,
// bqf, w2, b2, wp, bp, kc, vc, sqf, sw2, swp), in that order, 8 bytes each (the last three only for the W8A8 form).
extern "C" int mx_decode_mk_layer_bytes(void) { return (int)sizeof(MkLayer); }
