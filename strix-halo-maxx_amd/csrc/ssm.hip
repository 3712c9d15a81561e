// TRecViT recurrent block core on gfx950: temporal depthwise conv (4 taps) + block-diagonal input / decay gates +
// RG-LRU + the y-gate product, with torch's bf16 op-by-op rounding as restated in tapnext/npu/pack8.py:253-279
// (ssm_ref) and tapnext/npu/r9/cpuemu.py:33-47 (RGLRU.forward):
//
//   xc   = bf(bf(sum_fp32_{i=0..3} bf(x_{t-3+i} * w_i)) + b)           taps oldest .. current, zero before the video
//   gx   = bf(bf(xc_h Wx_h) + bx), ga = bf(bf(xc_h Wa_h) + ba)          per head h: 64 x 64 blocks (MFMA 32x32x16)
//   sx   = bf(sigmoid(gx)), sa = bf(sigmoid(ga))
//   loga = bf(bf(-8 sa) * sp)            sp = bf(softplus(a_param))
//   a    = bf(exp(loga)), g = bf(xc * sx)
//   first frame: h = g ;  else: mult = bf(sqrt(bf(1 - bf(exp(bf(2 loga)))))), h = a * h0 + bf(g * mult)   (fp32)
//   z    = bf(bf(h) * yg)
//
// Two forms:
//   mx_ssm_step  one streamed frame: h (fp32 state) updated in place, z written (the model.step contract)
//   mx_ssm_prep + mx_rglru_scan  a clip of F frames at once: prep writes the per-frame affine map h -> A h + B
//                (A = a, B = bf(g * mult); first frame A = 0, B = g) for every (frame, token, channel) in one launch,
//                then the scan runs the maps along time and writes z for every frame. Two scan kernels:
//                * chains (the clip shapes): one thread per (token, 4 channels) applies h = A h + B frame by frame,
//                  with the loads of 2 frames issued together; T C / 4 independent chains fill the GPU, every
//                  access is a coalesced stream, and h / z equal the streamed loop bit for bit (same operations in
//                  the same order);
//                * wave-parallel (too few chains to fill the GPU): one lane per frame, the maps composed with a
//                  64-lane shuffle scan (steps 1, 2, 4, .., 32); same h as the streamed loop up to fp32
//                  reassociation.
// RG-LRU form (mx_rglru_step, the RGLRU.forward(x, h0) -> (y, h) layer of tapnext/npu/r9/cpuemu.py:33-47 on its
// own): the conv and the y gate drop out (xc = x, y = bf(h)); the first frame is the host's h0 == null.
// Crop form (mx_ssm_step_rows, one streamed frame of a moving crop of patch tokens): token t's state lives in row
// rows[t] of the absolute state buffers (h, the history taps, the 32 x 32 patch grid + query rows), so the state
// moves with the image content and nothing is copied. Tokens that leave the crop drop their state and tokens that
// enter start from zero: per state row, a stamp (frame it entered the crop, last frame it was in the crop), double
// buffered by frame parity (read the previous frame's buffer, write this frame's), decides which state the row
// still has: h0 only if it was in the crop on the previous frame, history tap k only if it has been in the crop
// without a gap since frame t - k. The current frame's conv input is saved to its absolute row for later frames.
// Tile: a 1024-thread workgroup owns 64 tokens x one 64-channel head of one frame; the conv output tile is staged in
// LDS as the MFMA row operand; the gate weights are pre-transposed [head][out][in] so both operands are 16-byte lane
// reads; the gate sums go through LDS to the elementwise tail, which runs 4 consecutive channels of one token per
// thread (16- / 8-byte state, yg and z accesses).
#include "common.h"

namespace {

constexpr int XS = 72;  // LDS row stride of the conv tile (64 + 8)
constexpr int GS = 68;  // LDS row stride of the gate-sum tiles (fp32; 16-byte rows for the tail's vector reads)

// sigmoid and exp on the hardware exp2 / reciprocal (each within ~1 fp32 ulp, plus the rounding of x log2 e: a
// relative error below ~1e-6 over the gate and decay ranges, against the bf16 rounding (2^-9) every result takes
// next). The library expf and the IEEE division took several times the VALU work: TRecViT's streamed frame went
// 1.866-1.872 -> 1.845-1.847 ms with these.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float sigm(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_hw(-x)); }

struct SsmArgs {
  const uint16_t* tap[4];  // tap i (0 = current frame t, 1 = t-1, 2 = t-2, 3 = t-3) of frame 0 of the launch
  long ld_x;               // row stride of the tap matrices (elements)
  long fs_x;               // frame stride of the tap matrices (clip form)
  const uint16_t* yg; long ld_y; long fs_y;
  const uint16_t* conv_w;  // [4][C], row 0 = oldest tap (t-3)
  const uint16_t* conv_b;  // [C]
  const uint16_t* wxT; const uint16_t* bx;  // [H][64 out][64 in], [C]
  const uint16_t* waT; const uint16_t* ba;
  const uint16_t* sp;      // [C] bf16(softplus(a_param))
  const int* frame;        // global index of frame 0 of this launch (first frame of the video <=> index 0)
  float* h; long fs_h;     // fp32 state [T][C] (step form) / unused (prep form)
  const float* h0;         // the state read before the update (== h except in the RG-LRU form)
  int first;               // RG-LRU form: 1 = first frame (no h0), in place of the device frame counter
  uint16_t* z; long ld_z; long fs_z;
  float* A; float* B; long fs_ab;  // prep form outputs [F][T][C]
  int T, C, mode;          // mode 0 = step, 1 = prep
  // crop form (rows != nullptr): token -> state row; stamps [2][srows] {entered, last present}; xsave: this frame's
  // ring slot (absolute rows, stride ld_save) that receives the current conv input
  const int* rows; int2* stamps; int srows; uint16_t* xsave; long ld_save;
};

// The crop form's view of one state row at frame tnow: fresh = not in the crop on frame tnow - 1; enter = frame it
// entered the crop (tnow when fresh).
__device__ __forceinline__ void row_stamp(const SsmArgs& p, int row, int tnow, bool& fresh, int& enter) {
  const int2 s = p.stamps[((tnow - 1) & 1) * p.srows + row];
  fresh = s.y != tnow - 1;
  enter = fresh ? tnow : s.x;
}

// RG: the RG-LRU form (no conv, no y gate, first frame from p.first).
// 1024 threads (16 waves) per 64-token x 64-channel tile. The conv tile goes to LDS (512 threads, one 8-channel item
// each); waves 0-3 run the gate products (MFMA 32x32x16, wave -> 32 tokens x 32 channels) and leave the raw fp32
// sums in LDS; then all 1024 threads run the elementwise RG-LRU tail on 4 (token, channel) elements each: thread ->
// token tid / 16, channels 4 (tid % 16) .. + 3, so the state / yg / z accesses are 16- / 8-byte vectors and each
// thread's serial chain of transcendentals is 4 elements long, with 4 waves per SIMD to hide its latency.
template <bool RG>
__global__ __launch_bounds__(1024) void ssm_kernel(SsmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[64 * XS];
  __shared__ __attribute__((aligned(16))) float gsh[2][64 * GS];  // gate sums [token][channel], x then a
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, hk = lane >> 5;
  const int t0 = blockIdx.x * 64, q = blockIdx.y, f = blockIdx.z;
  const int c0 = q * 64;
  const int tnow = RG ? (p.first ? 0 : 1) : *p.frame + f;
  const bool first = tnow == 0;
  // tail element group of this thread
  const int tl = tid >> 4, cl = (tid & 15) * 4;
  const int token = t0 + tl, tok_c = min(token, p.T - 1);
  // the gate products' weight fragments (waves 0-3: wave -> tm = token half, tn = channel half), issued first
  const int tm = (wave >> 1) & 1, tn = wave & 1;
  u32x4 wxf[4], waf[4];
  if (wave < 4) {
    const uint16_t* wxr = p.wxT + ((long)q * 64 + tn * 32 + lr) * 64;
    const uint16_t* war = p.waT + ((long)q * 64 + tn * 32 + lr) * 64;
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      wxf[s4] = *reinterpret_cast<const u32x4*>(wxr + 16 * s4 + 8 * hk);
      waf[s4] = *reinterpret_cast<const u32x4*>(war + 16 * s4 + 8 * hk);
    }
  }
  // per-channel RG-LRU parameters of the thread's 4 channels (held as packed bf16 pairs)
  const u32x2 spw = *reinterpret_cast<const u32x2*>(p.sp + c0 + cl);
  const u32x2 bxw = *reinterpret_cast<const u32x2*>(p.bx + c0 + cl);
  const u32x2 baw = *reinterpret_cast<const u32x2*>(p.ba + c0 + cl);

  // ---- step form: the state row and yg of the thread's 4 elements, loaded first (their latency runs under the conv
  // and the gate products). Clamped indices, no branch around the loads; which of them count (token < T, first frame,
  // fresh crop row) is applied where the values are used. The crop form's row map and stamp are dependent rounds.
  f32x4 hraw = {0.f, 0.f, 0.f, 0.f};
  u32x2 yraw = {0x3f803f80u, 0x3f803f80u};  // bf16 1.0 pairs: the RG-LRU form's z = bf(h)
  int rw = tok_c;                            // state row of the thread's token
  bool fresh = false;                        // its crop row was not in the crop on the previous frame (state 0)
  if (p.mode == 0) {
    if (p.rows) {
      rw = min(max(p.rows[tok_c], 0), p.srows - 1);
      if (!first) {
        int enter;
        row_stamp(p, rw, tnow, fresh, enter);
      }
    }
    if (!(RG && first)) hraw = *reinterpret_cast<const f32x4*>(p.h0 + (long)rw * p.C + c0 + cl);
    if (!RG) yraw = *reinterpret_cast<const u32x2*>(p.yg + f * p.fs_y + (long)tok_c * p.ld_y + c0 + cl);
  }

  // ---- temporal conv of the 64 x 64 tile into LDS: threads 0-511, one 8-channel item each
  if (tid < 512) {
    const int tok = tid >> 3, cc = (tid & 7) * 8;
    const int tk = min(t0 + tok, p.T - 1);
    const int row = p.rows ? min(max(p.rows[tk], 0), p.srows - 1) : tk;  // clamped: never out of bounds
    int ntap = (first || RG) ? 1 : 4;  // taps 0 .. ntap - 1 carry data; the older ones are zero
    int enter = tnow;
    if (p.rows && !first) {
      bool fr;
      row_stamp(p, row, tnow, fr, enter);
      ntap = fr ? 1 : min(4, tnow - enter + 1);  // tap k (frame tnow - k) needs enter <= tnow - k
    }
    u32x4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      u32x4 v = {0u, 0u, 0u, 0u};
      const long r = i == 0 ? tk : row;  // the current frame's rows are the launch's tokens
      if (i < ntap) v = *reinterpret_cast<const u32x4*>(p.tap[i] + f * p.fs_x + r * p.ld_x + c0 + cc);
      xv[i] = v;
    }
    u32x4 bb = {0u, 0u, 0u, 0u};
    u32x4 w[4] = {bb, bb, bb, bb};
    if (!RG) {
      bb = *reinterpret_cast<const u32x4*>(p.conv_b + c0 + cc);
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = *reinterpret_cast<const u32x4*>(p.conv_w + i * p.C + c0 + cc);
    }
    if (p.rows && t0 + tok < p.T) {
      *reinterpret_cast<u32x4*>(p.xsave + (long)row * p.ld_save + c0 + cc) = xv[0];
      if (q == 0 && cc == 0) p.stamps[(tnow & 1) * p.srows + row] = make_int2(enter, tnow);
    }
    u32x4 o = xv[0];  // RG-LRU form: xc = x
#pragma unroll
    for (int e = 0; e < 4 && !RG; e++) {
      float r[2];
#pragma unroll
      for (int hl = 0; hl < 2; hl++) {
        auto get = [&](u32x4 v) { return hl ? hi_bf(v[e]) : lo_bf(v[e]); };
        // w row i = tap (t-3+i): oldest first; xv index 3-i holds frame t-3+i
        float sum = rbf(get(xv[3]) * get(w[0]));
        sum = sum + rbf(get(xv[2]) * get(w[1]));
        sum = sum + rbf(get(xv[1]) * get(w[2]));
        sum = sum + rbf(get(xv[0]) * get(w[3]));
        r[hl] = rbf(sum) + get(bb);
      }
      o[e] = pack2(r[0], r[1]);
    }
    *reinterpret_cast<u32x4*>(&xs[tok * XS + cc]) = o;
  }
  __syncthreads();

  // ---- gates: waves 0-3 -> 32 tokens (tm) x 32 output channels (tn) of both gates; raw fp32 sums to LDS
  if (wave < 4) {
    f32x16 gx, ga;
#pragma unroll
    for (int e = 0; e < 16; e++) { gx[e] = 0.f; ga[e] = 0.f; }
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int k = 16 * s + 8 * hk;
      const bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(&xs[(tm * 32 + lr) * XS + k]));
      gx = mfma32(a, as_bf16x8(wxf[s]), gx);
      ga = mfma32(a, as_bf16x8(waf[s]), ga);
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int tr = tm * 32 + 8 * (r >> 2) + 4 * hk + (r & 3);
      gsh[0][tr * GS + tn * 32 + lr] = gx[r];
      gsh[1][tr * GS + tn * 32 + lr] = ga[r];
    }
  }
  __syncthreads();

  // ---- elementwise RG-LRU: 4 channels of one token per thread
  if (token >= p.T) return;
  const f32x4 gxv = *reinterpret_cast<const f32x4*>(&gsh[0][tl * GS + cl]);
  const f32x4 gav = *reinterpret_cast<const f32x4*>(&gsh[1][tl * GS + cl]);
  const u32x2 xcw = *reinterpret_cast<const u32x2*>(&xs[tl * XS + cl]);
  f32x4 hv, Av, Bv;
  float zv[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t pick = (e >> 1) ? 1 : 0;
    auto half = [&](const u32x2& w) { return (e & 1) ? hi_bf(pick ? w.y : w.x) : lo_bf(pick ? w.y : w.x); };
    const float xcv = half(xcw), spc = half(spw), bxc = half(bxw), bac = half(baw);
    const float gxp = rbf(rbf(gxv[e]) + bxc), gap = rbf(rbf(gav[e]) + bac);
    const float sx = rbf(sigm(gxp)), sa = rbf(sigm(gap));
    const float loga = rbf(rbf(-8.0f * sa) * spc);
    const float av = rbf(exp_hw(loga));
    const float g = rbf(xcv * sx);
    float Am, Bm;
    if (first) {
      Am = 0.f;
      Bm = g;
    } else {
      const float e2 = rbf(exp_hw(rbf(2.0f * loga)));
      const float mult = rbf(sqrtf(rbf(1.0f - e2)));
      Am = av;
      Bm = rbf(g * mult);
    }
    const float hp = fresh ? 0.f : hraw[e];  // a fresh crop row starts from 0
    const float h = first ? g : __fadd_rn(__fmul_rn(Am, hp), Bm);
    hv[e] = h;
    zv[e] = rbf(h) * half(yraw);
    Av[e] = Am;
    Bv[e] = Bm;
  }
  if (p.mode == 0) {
    *reinterpret_cast<f32x4*>(p.h + (long)rw * p.C + c0 + cl) = hv;
    *reinterpret_cast<u32x2*>(p.z + f * p.fs_z + (long)token * p.ld_z + c0 + cl) =
        u32x2{pack2(zv[0], zv[1]), pack2(zv[2], zv[3])};
  } else {
    const long idx = (long)token * p.C + c0 + cl;
    *reinterpret_cast<f32x4*>(p.A + f * p.fs_ab + idx) = Av;
    *reinterpret_cast<f32x4*>(p.B + f * p.fs_ab + idx) = Bv;
  }
}

// ---- time scan: h_t = A_t h_{t-1} + B_t for every (token, channel), frames on the lanes of a wave
constexpr int SC = 64;  // channels per workgroup

__global__ __launch_bounds__(256) void rglru_scan_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                         long fs_ab, float* __restrict__ h, int F, int C,
                                                         const uint16_t* __restrict__ yg, long ld_y, long fs_y,
                                                         uint16_t* __restrict__ z, long ld_z, long fs_z) {
  __shared__ float sa[64][SC + 1];
  __shared__ float sb[64][SC + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = blockIdx.x * SC, token = blockIdx.y;
  const int T = gridDim.y;
  (void)T;
  // carried state for this wave's 16 channels: lane j < 16 of each wave holds channel wave*16 + j
  float carry = 0.f;
  if (lane < 16 && c0 + wave * 16 + lane < C) carry = h[(long)token * C + c0 + wave * 16 + lane];
  for (int f0 = 0; f0 < F; f0 += 64) {
    const int nf = min(64, F - f0);
    __syncthreads();
    // coalesced tile load: rows = frames, 64 channels each
    for (int i = tid; i < 64 * SC; i += 256) {
      const int fr = i / SC, cc = i % SC;
      float av = 1.f, bv = 0.f;  // identity map beyond the clip
      if (fr < nf && c0 + cc < C) {
        const long o = (long)(f0 + fr) * fs_ab + (long)token * C + c0 + cc;
        av = A[o];
        bv = B[o];
      }
      sa[fr][cc] = av;
      sb[fr][cc] = bv;
    }
    __syncthreads();
    // each wave scans 16 channels, one at a time: lane = frame
    for (int j = 0; j < 16; j++) {
      const int cc = wave * 16 + j;
      float a = sa[lane][cc], b = sb[lane][cc];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float ap = __shfl_up(a, d, 64), bp = __shfl_up(b, d, 64);
        if (lane >= d) {
          b = __fadd_rn(__fmul_rn(a, bp), b);
          a = __fmul_rn(a, ap);
        }
      }
      const float c_in = __shfl(carry, j, 64);
      const float hv = __fadd_rn(__fmul_rn(a, c_in), b);
      sb[lane][cc] = hv;
      const float last = __shfl(hv, nf - 1, 64);
      if (lane == j) carry = last;
    }
    __syncthreads();
    // z = bf(bf(h) * yg) for the tile, coalesced along channels
    for (int i = tid; i < 64 * SC; i += 256) {
      const int fr = i / SC, cc = i % SC;
      if (fr < nf && c0 + cc < C) {
        const long f = f0 + fr;
        const float yv = bf2f(yg[f * fs_y + (long)token * ld_y + c0 + cc]);
        z[f * fs_z + (long)token * ld_z + c0 + cc] = f2bf(rbf(sb[fr][cc]) * yv);
      }
    }
  }
  if (lane < 16 && c0 + wave * 16 + lane < C) h[(long)token * C + c0 + wave * 16 + lane] = carry;
}

// ---- chain scan: thread = (token, 4 consecutive channels), frames in order
constexpr int CHF = 2;   // frames whose loads are issued before their arithmetic (2-4 measured best: occupancy)
constexpr int ZB = 16;   // frames whose z stay in registers until one burst of stores after them

// The loads of A and B and the stores of z are non-temporal (each byte is touched once), and the z of ZB frames are
// stored together after their recurrence steps instead of one frame at a time between the next frames' loads: the
// HBM then serves long runs of reads and of writes (16 frames, 1280 x 768: 38.3 -> 36.6 us per launch; with plain
// stores the late burst is slower, 41.7 us).
__global__ __launch_bounds__(256) void rglru_chain_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                          long fs_ab, float* __restrict__ h, int F, int T, int C,
                                                          const uint16_t* __restrict__ yg, long ld_y, long fs_y,
                                                          uint16_t* __restrict__ z, long ld_z, long fs_z) {
  const int c4n = C >> 2;
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i >= (long)T * c4n) return;
  const int t = (int)(i / c4n), c = (int)(i % c4n) * 4;
  const long o = (long)t * C + c;
  f32x4 hv = *reinterpret_cast<const f32x4*>(h + o);
  for (int f1 = 0; f1 < F; f1 += ZB) {
    u32x2 zs[ZB];
#pragma unroll
    for (int f0 = 0; f0 < ZB; f0 += CHF) {
      f32x4 av[CHF], bv[CHF];
      u32x2 yv[CHF];
#pragma unroll
      for (int k = 0; k < CHF; k++) {  // frames past F reload the last one (never applied, never stored)
        const long f = min(f1 + f0 + k, F - 1);
        av[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(A + f * fs_ab + o));
        bv[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(B + f * fs_ab + o));
        yv[k] = *reinterpret_cast<const u32x2*>(yg + f * fs_y + (long)t * ld_y + c);
      }
#pragma unroll
      for (int k = 0; k < CHF; k++) {
        if (f1 + f0 + k < F) {
#pragma unroll
          for (int e = 0; e < 4; e++) hv[e] = __fadd_rn(__fmul_rn(av[k][e], hv[e]), bv[k][e]);
        }
        zs[f0 + k] = u32x2{pack2(rbf(hv[0]) * lo_bf(yv[k].x), rbf(hv[1]) * hi_bf(yv[k].x)),
                           pack2(rbf(hv[2]) * lo_bf(yv[k].y), rbf(hv[3]) * hi_bf(yv[k].y))};
      }
    }
#pragma unroll
    for (int f = 0; f < ZB; f++)
      if (f1 + f < F)
        __builtin_nontemporal_store(zs[f], reinterpret_cast<u32x2*>(z + (long)(f1 + f) * fs_z + (long)t * ld_z + c));
  }
  *reinterpret_cast<f32x4*>(h + o) = hv;
}

int check_common(const SsmArgs& p, int F) {
  for (int i = 0; i < 4; i++)
    if (!p.tap[i]) return MX_ENULL;
  if (!p.conv_w || !p.conv_b || !p.wxT || !p.bx || !p.waT || !p.ba || !p.sp || !p.frame) return MX_ENULL;
  if (p.T < 1 || F < 1 || p.C % 64 || p.ld_x % 8 || p.C > 65535 * 64) return MX_ESHAPE;
  for (int i = 0; i < 4; i++)
    if ((uintptr_t)p.tap[i] & 15) return MX_ELAYOUT;
  if (((uintptr_t)p.conv_w | (uintptr_t)p.conv_b | (uintptr_t)p.wxT | (uintptr_t)p.waT) & 15) return MX_ELAYOUT;
  if (((uintptr_t)p.sp | (uintptr_t)p.bx | (uintptr_t)p.ba) & 7) return MX_ELAYOUT;  // 4-channel vector reads
  return MX_OK;
}

// The step / RG-LRU forms' per-element operands, read and written as 4-channel vectors: fp32 state rows 16-byte
// aligned, yg / z rows 8-byte aligned with strides of whole 4-element groups.
int check_step_io(const float* h, const float* h0, const uint16_t* yg, long ld_y, const uint16_t* z, long ld_z) {
  if (((uintptr_t)h | (uintptr_t)h0) & 15) return MX_ELAYOUT;
  if (yg && (((uintptr_t)yg & 7) || ld_y % 4)) return MX_ELAYOUT;
  if (((uintptr_t)z & 7) || ld_z % 4) return MX_ELAYOUT;
  return MX_OK;
}

}  // namespace

// One streamed frame. taps: current frame x_t and the three previous frames (rows of width >= C, stride ld_x);
// h [T][C] fp32 updated in place; z [T][ld_z] bf16; yg [T][ld_y] bf16; frame: device int, 0 = first frame.
extern "C" int mx_ssm_step(hipStream_t st, const uint16_t* x0, const uint16_t* x1, const uint16_t* x2,
                           const uint16_t* x3, long ld_x, const uint16_t* yg, long ld_y, const uint16_t* conv_w,
                           const uint16_t* conv_b, const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT,
                           const uint16_t* ba, const uint16_t* sp, const int* frame, float* h, uint16_t* z, long ld_z,
                           int T, int C) {
  SsmArgs p{{x0, x1, x2, x3}, ld_x, 0, yg, ld_y, 0, conv_w, conv_b, wxT, bx, waT, ba, sp, frame, h, 0, h, 0,
            z, ld_z, 0, nullptr, nullptr, 0, T, C, 0, nullptr, nullptr, 0, nullptr, 0};
  int rc = check_common(p, 1);
  if (rc) return rc;
  if (!yg || !h || !z) return MX_ENULL;
  rc = check_step_io(h, h, yg, ld_y, z, ld_z);
  if (rc) return rc;
  hipLaunchKernelGGL(ssm_kernel<false>, dim3((T + 63) / 64, C / 64, 1), dim3(1024), 0, st, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// One streamed frame of a moving crop: T tokens (crop patches, then queries); x0 / yg / z: the launch's token rows;
// x1..x3 (history, stride ld_x), h (fp32 [srows][C]) and xsave (this frame's history slot, stride ld_save):
// absolute state rows, token t at rows[t] (distinct, < srows); stamps: [2][srows] int pairs, {-8, -8} after a reset.
extern "C" int mx_ssm_step_rows(hipStream_t st, const uint16_t* x0, const uint16_t* x1, const uint16_t* x2,
                                const uint16_t* x3, long ld_x, const uint16_t* yg, long ld_y, const uint16_t* conv_w,
                                const uint16_t* conv_b, const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT,
                                const uint16_t* ba, const uint16_t* sp, const int* frame, float* h, uint16_t* z,
                                long ld_z, int T, int C, const int* rows, int* stamps, int srows, uint16_t* xsave,
                                long ld_save) {
  SsmArgs p{{x0, x1, x2, x3}, ld_x, 0, yg, ld_y, 0, conv_w, conv_b, wxT, bx, waT, ba, sp, frame, h, 0, h, 0,
            z, ld_z, 0, nullptr, nullptr, 0, T, C, 0, rows, reinterpret_cast<int2*>(stamps), srows, xsave, ld_save};
  int rc = check_common(p, 1);
  if (rc) return rc;
  if (!yg || !h || !z || !rows || !stamps || !xsave) return MX_ENULL;
  if (srows < T || ld_save % 8 || ((uintptr_t)xsave & 15) || ((uintptr_t)stamps & 7)) return MX_ESHAPE;
  rc = check_step_io(h, h, yg, ld_y, z, ld_z);
  if (rc) return rc;
  hipLaunchKernelGGL(ssm_kernel<false>, dim3((T + 63) / 64, C / 64, 1), dim3(1024), 0, st, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// The RG-LRU layer alone (tapnext/npu/r9/cpuemu.py:33-47, RGLRU.forward(x, h0) -> (y, h)): x [T][ld_x] bf16 (the
// conv output the layer receives), h0 [T][C] fp32 or null for the first frame (h = x * sigmoid(gate_x)), h [T][C]
// fp32 written (may be h0: in place), y [T][ld_y] = bf16(h).
extern "C" int mx_rglru_step(hipStream_t st, const uint16_t* x, long ld_x, const float* h0, const uint16_t* wxT,
                             const uint16_t* bx, const uint16_t* waT, const uint16_t* ba, const uint16_t* sp, float* h,
                             uint16_t* y, long ld_y, int T, int C) {
  if (!x || !wxT || !bx || !waT || !ba || !sp || !h || !y) return MX_ENULL;
  if (T < 1 || C % 64 || C > 65535 * 64 || ld_x % 8 || ld_x < C || ld_y < C || T > 65535 * 64) return MX_ESHAPE;
  if (((uintptr_t)x | (uintptr_t)wxT | (uintptr_t)waT) & 15) return MX_ELAYOUT;
  if (((uintptr_t)sp | (uintptr_t)bx | (uintptr_t)ba) & 7) return MX_ELAYOUT;
  const int rc = check_step_io(h, h0 ? h0 : h, nullptr, 0, y, ld_y);
  if (rc) return rc;
  SsmArgs p{{x, x, x, x}, ld_x, 0, nullptr, 0, 0, nullptr, nullptr, wxT, bx, waT, ba, sp, nullptr, h, 0, h0,
            h0 ? 0 : 1, y, ld_y, 0, nullptr, nullptr, 0, T, C, 0, nullptr, nullptr, 0, nullptr, 0};
  hipLaunchKernelGGL(ssm_kernel<true>, dim3((T + 63) / 64, C / 64, 1), dim3(1024), 0, st, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Clip form, part 1: F frames at once. x_stack holds F + 3 frames of the conv input (frame stride fs_x; the first 3
// are the history before the clip, zero at the start of a video); A, B: [F][T][C] fp32 outputs.
extern "C" int mx_ssm_prep(hipStream_t st, const uint16_t* x_stack, long ld_x, long fs_x, const uint16_t* conv_w,
                           const uint16_t* conv_b, const uint16_t* wxT, const uint16_t* bx, const uint16_t* waT,
                           const uint16_t* ba, const uint16_t* sp, const int* frame, float* A, float* B, int F, int T,
                           int C) {
  SsmArgs p{{x_stack + 3 * fs_x, x_stack + 2 * fs_x, x_stack + fs_x, x_stack}, ld_x, fs_x, nullptr, 0, 0, conv_w,
            conv_b, wxT, bx, waT, ba, sp, frame, nullptr, 0, nullptr, 0, nullptr, 0, 0, A, B, (long)T * C, T, C, 1,
            nullptr, nullptr, 0, nullptr, 0};
  int rc = check_common(p, F);
  if (rc) return rc;
  if (!A || !B) return MX_ENULL;
  if (fs_x % 8 || F > 65535) return MX_ESHAPE;
  if (((uintptr_t)A | (uintptr_t)B) & 15) return MX_ELAYOUT;
  hipLaunchKernelGGL(ssm_kernel<false>, dim3((T + 63) / 64, C / 64, F), dim3(1024), 0, st, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

// Clip form, part 2: h (fp32 [T][C], state before the clip, updated to the state after it); z for every frame.
extern "C" int mx_rglru_scan(hipStream_t st, const float* A, const float* B, float* h, int F, int T, int C,
                             const uint16_t* yg, long ld_y, long fs_y, uint16_t* z, long ld_z, long fs_z) {
  if (!A || !B || !h || !yg || !z) return MX_ENULL;
  if (F < 1 || T < 1 || T > 65535 || C % 64) return MX_ESHAPE;
  // chains when they fill the GPU (>= 64 K of them: 256 CUs x 256 threads) and the rows allow 16 / 8-byte accesses
  const long chains = (long)T * C / 4;
  const bool aligned = !(((uintptr_t)A | (uintptr_t)B | (uintptr_t)h) & 15) && !(((uintptr_t)yg | (uintptr_t)z) & 7) &&
                       ld_y % 4 == 0 && fs_y % 4 == 0 && ld_z % 4 == 0 && fs_z % 4 == 0;
  if (chains >= 65536 && aligned)
    hipLaunchKernelGGL(rglru_chain_kernel, dim3((unsigned)((chains + 255) / 256)), dim3(256), 0, st, A, B,
                       (long)T * C, h, F, T, C, yg, ld_y, fs_y, z, ld_z, fs_z);
  else
    hipLaunchKernelGGL(rglru_scan_kernel, dim3(C / SC, T), dim3(256), 0, st, A, B, (long)T * C, h, F, C, yg, ld_y,
                       fs_y, z, ld_z, fs_z);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
