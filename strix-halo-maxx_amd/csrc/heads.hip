// TAPNext tracking heads (coordinate head + visibility head) on the encoder-normed query tokens, with the
// coordinate head's windowed soft-argmax readout, all in fp32.
//
// Each head is Linear(D -> H), LayerNorm, GELU (erf), Linear(H -> H), LayerNorm, GELU (erf), Linear(H -> NO). The
// coordinate head's NO = 2n logits are two n-bin distributions (first half, then second half); each is read out as
// the expectation of the bin index under softmax(0.5 * logits) restricted to bins within `radius` of the argmax
// (first index among equal maxima), plus 0.5. The visibility head's single output is the visibility logit.
//
// Layout: one workgroup of 512 threads (8 waves) per (pair of query rows, head). The query rows are staged in LDS as
// fp32. In a hidden layer, thread t owns hidden unit j = t % 256 (H <= 256) for the k half t / 256 and walks the
// transposed weights W^T[k][j] of that half with 16 loads in flight, so every weight load is a coalesced row of W^T
// shared by the workgroup's QB query rows; the halves' sums meet in LDS (half 0 + half 1). The output Linear gives
// each thread one output column over the whole K (the single visibility output: a block reduction). Two waves per
// SIMD keep the load latency of one under the other's work. Sums run in a fixed order (k ascending within a half,
// then the halves; lanes then waves for the reductions), so the result does not depend on the launch.
//
// Weight blob of one head (fp32, contiguous):
//   W0T [D][H] | b0 [H] | g0 [H] | beta0 [H] | W1T [H][H] | b1 [H] | g1 [H] | beta1 [H] | W2T [H][NO] | b2 [NO]
#include "common.h"

namespace {

constexpr int NT = 512;       // threads per workgroup (8 waves: measured 54 us per frame's heads, 4 waves 75, 16 waves 80)
constexpr int NWV = NT / 64;  // waves per workgroup
constexpr int HU = 256;       // hidden units per k part (the hidden width is at most HU)
constexpr int NP = NT / HU;   // k parts of a hidden layer
constexpr int QB = 2;         // query rows per workgroup
constexpr int KU = 16;        // weight loads a thread issues before their products

// Block-wide sums of QB values per thread (every thread gets the totals). red: NWV waves x QB floats of LDS.
__device__ __forceinline__ void block_sum(float (&v)[QB], float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int r = 0; r < QB; r++) v[r] = wave_sum(v[r]);
  __syncthreads();
  if (lane == 0)
#pragma unroll
    for (int r = 0; r < QB; r++) red[w * QB + r] = v[r];
  __syncthreads();
#pragma unroll
  for (int r = 0; r < QB; r++) {
    float t = red[r];
#pragma unroll
    for (int ww = 1; ww < NWV; ww++) t = t + red[ww * QB + r];
    v[r] = t;
  }
}

// acc[r] += sum over k in [k0, k1) of x[r][k] W^T[k][col], k ascending, KU loads issued ahead of their products.
__device__ __forceinline__ void dot_col(const float* x, int ldxs, int k0, int k1, const float* __restrict__ WT, long ldw,
                                        int col, float (&acc)[QB]) {
  for (int k = k0; k < k1; k += KU) {
    float w[KU];
#pragma unroll
    for (int u = 0; u < KU; u++) w[u] = WT[(long)(k + u) * ldw + col];
#pragma unroll
    for (int u = 0; u < KU; u++)
#pragma unroll
      for (int r = 0; r < QB; r++) acc[r] = acc[r] + x[r * ldxs + k + u] * w[u];
  }
}

// y[r][j] = GELU(LN(sum_k x[r][k] W^T[k][j] + b[j])) for j < H, r < QB; x and y in LDS. part: LDS for the k parts
// 1 .. NP - 1's partial sums ([NP - 1][QB][HU]), added to part 0's in part order.
__device__ void dense_ln_gelu(const float* x, int ldxs, int K, const float* __restrict__ WT, const float* b,
                              const float* g, const float* be, float eps, int H, float* y, int ldys, float* red,
                              float* part) {
  const int j = threadIdx.x % HU, kp = threadIdx.x / HU;
  float acc[QB];
#pragma unroll
  for (int r = 0; r < QB; r++) acc[r] = 0.f;
  if (j < H) dot_col(x, ldxs, kp * (K / NP), (kp + 1) * (K / NP), WT, H, j, acc);
  if (kp > 0 && j < H)
#pragma unroll
    for (int r = 0; r < QB; r++) part[((kp - 1) * QB + r) * HU + j] = acc[r];
  __syncthreads();
  const bool mine = kp == 0 && j < H;
  if (mine)
#pragma unroll
    for (int r = 0; r < QB; r++) {
#pragma unroll
      for (int q = 1; q < NP; q++) acc[r] = acc[r] + part[((q - 1) * QB + r) * HU + j];
      acc[r] = acc[r] + b[j];
    }
  float s[QB];
#pragma unroll
  for (int r = 0; r < QB; r++) s[r] = mine ? acc[r] : 0.f;
  block_sum(s, red);
  float mu[QB], d[QB];
#pragma unroll
  for (int r = 0; r < QB; r++) {
    mu[r] = s[r] / (float)H;
    d[r] = mine ? (acc[r] - mu[r]) * (acc[r] - mu[r]) : 0.f;
  }
  block_sum(d, red);
  if (mine) {
#pragma unroll
    for (int r = 0; r < QB; r++) {
      const float var = d[r] / (float)H;
      const float hn = (acc[r] - mu[r]) / sqrtf(var + eps) * g[j] + be[j];
      y[r * ldys + j] = gelu_erf(hn);
    }
  }
  __syncthreads();
}

// (max value, first index) over the block; ties go to the smaller index.
__device__ __forceinline__ void arg_better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

__global__ void __launch_bounds__(NT) track_heads_kernel(
    const uint16_t* __restrict__ x, long ldx, int Q, int D, int H, const float* __restrict__ cblob, int NOC,
    float ce0, float ce1, const float* __restrict__ vblob, float ve0, float ve1, int radius,
    float* __restrict__ tracks, float* __restrict__ logits, long ldl, float* __restrict__ vis) {
  extern __shared__ float sm[];
  const int head = blockIdx.y, tid = threadIdx.x;
  const int q0 = blockIdx.x * QB, nr = min(QB, Q - q0);
  const int NO = head ? 1 : NOC;
  const float* blob = head ? vblob : cblob;
  const float e0 = head ? ve0 : ce0, e1 = head ? ve1 : ce1;
  float* xs = sm;                   // [QB][D]
  float* h0 = xs + QB * D;          // [QB][H]
  float* h1 = h0 + QB * H;          // [QB][H]
  float* os = h1 + QB * H;          // [QB][NOC]
  float* part = os + QB * NOC;      // [NP - 1][QB][HU] k-part partial sums
  float* red = part + (NP - 1) * QB * HU;  // [NWV][QB] (sums), then [NWV] argmax indices
  for (int e = tid; e < QB * D; e += NT) {
    const int r = e / D, k = e - r * D;
    xs[e] = r < nr ? bf2f(x[(long)(q0 + r) * ldx + k]) : 0.f;
  }
  __syncthreads();
  const float* W0 = blob;
  const float *b0 = W0 + (long)D * H, *g0 = b0 + H, *be0 = g0 + H;
  const float* W1 = be0 + H;
  const float *b1 = W1 + (long)H * H, *g1 = b1 + H, *be1 = g1 + H;
  const float* W2 = be1 + H;
  const float* b2 = W2 + (long)H * NO;
  dense_ln_gelu(xs, D, D, W0, b0, g0, be0, e0, H, h0, H, red, part);
  dense_ln_gelu(h0, H, H, W1, b1, g1, be1, e1, H, h1, H, red, part);
  if (head) {
    // the one visibility output: thread k < H holds the product of hidden unit k, summed over the block
    float pv[QB];
#pragma unroll
    for (int r = 0; r < QB; r++) pv[r] = tid < H ? h1[r * H + tid] * W2[tid] : 0.f;
    block_sum(pv, red);
#pragma unroll
    for (int r = 0; r < QB; r++)
      if (tid == r && r < nr) vis[q0 + r] = pv[r] + b2[0];
    return;
  }
  for (int o = tid; o < NO; o += NT) {
    float acc[QB];
#pragma unroll
    for (int r = 0; r < QB; r++) acc[r] = 0.f;
    dot_col(h1, H, 0, H, W2, NO, o, acc);
#pragma unroll
    for (int r = 0; r < QB; r++) os[r * NOC + o] = acc[r] + b2[o];
  }
  __syncthreads();
  for (int e = tid; e < nr * NOC; e += NT) {
    const int r = e / NOC, o = e - r * NOC;
    logits[(long)(q0 + r) * ldl + o] = os[r * NOC + o];
  }
  // ---- windowed soft-argmax of each n-bin half, one (row, half) at a time
  const int n = NOC / 2, lane = tid & 63, w = tid >> 6;
  float* redi = red + NWV * QB;
  for (int r = 0; r < nr; r++) {
    for (int half = 0; half < 2; half++) {
      const float* z = os + r * NOC + half * n;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = tid; i < n; i += NT) arg_better(bv, bi, z[i], i);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float v2 = __shfl_xor(bv, off, 64);
        const int i2 = __shfl_xor(bi, off, 64);
        arg_better(bv, bi, v2, i2);
      }
      __syncthreads();
      if (lane == 0) { red[w] = bv; redi[w] = __int_as_float(bi); }
      __syncthreads();
      float mv = red[0];
      int am = __float_as_int(redi[0]);
      for (int ww = 1; ww < NWV; ww++) arg_better(mv, am, red[ww], __float_as_int(redi[ww]));
      const float zmax = 0.5f * mv;
      // softmax over all n bins, then the window mask, then renormalised (the order of the readout's definition)
      float es[2], s1[QB] = {}, s2[QB] = {}, s3[QB] = {};
      for (int u = 0; u < 2; u++) {
        const int i = tid + u * NT;
        es[u] = i < n ? expf(0.5f * z[i] - zmax) : 0.f;
        s1[0] += es[u];
      }
      block_sum(s1, red);
      float pr[2];
      for (int u = 0; u < 2; u++) {
        const int i = tid + u * NT;
        const bool in = i < n && abs(am - i) <= radius;
        pr[u] = in ? es[u] / s1[0] : 0.f;
        s2[0] += pr[u];
      }
      block_sum(s2, red);
      for (int u = 0; u < 2; u++) {
        const int i = tid + u * NT;
        s3[0] += (pr[u] / s2[0]) * (float)i;
      }
      block_sum(s3, red);
      if (tid == 0) tracks[(long)(q0 + r) * 2 + half] = s3[0] + 0.5f;
      __syncthreads();
    }
  }
}

}  // namespace

// Floats in one head's weight blob (layout above).
extern "C" long mx_track_head_blob_elems(int D, int H, int NO) {
  return (long)D * H + 3L * H + (long)H * H + 3L * H + (long)H * NO + NO;
}

// x: Q encoder-normed query rows (bf16, row stride ldx >= D). cblob: coordinate head (NO = NOC = 2n logits, n <= 512
// bins per coordinate), vblob: visibility head (NO = 1). e*: the four LayerNorm eps. Outputs fp32: tracks (Q, 2)
// (half 0, half 1 readouts), logits (Q, NOC) with row stride ldl, vis (Q).
extern "C" int mx_track_heads(hipStream_t st, const uint16_t* x, long ldx, int Q, int D, int H, const float* cblob,
                              int NOC, float ce0, float ce1, const float* vblob, float ve0, float ve1, int radius,
                              float* tracks, float* logits, long ldl, float* vis) {
  // H <= 256: one hidden unit per thread of a k part; D, H multiples of 32: whole KU groups in each of the 2 k parts;
  // NOC <= 512: one output column per thread, at most 2 bins per thread in the readout
  if (Q < 0 || D < 64 || D > 4096 || D % (KU * NP) || H < 64 || H > HU || H % (KU * NP) || NOC < 2 || NOC % 2 ||
      NOC > 512 || radius < 0 || ldx < D || ldl < NOC)
    return MX_ESHAPE;
  if (Q == 0) return MX_OK;
  if (!x || !cblob || !vblob || !tracks || !logits || !vis) return MX_ENULL;
  const size_t smem =
      sizeof(float) * ((size_t)QB * D + 2 * QB * H + (size_t)QB * NOC + (NP - 1) * QB * HU + 2 * NWV * QB);
  if (smem > 160 * 1024) return MX_ESHAPE;
  hipLaunchKernelGGL(track_heads_kernel, dim3((Q + QB - 1) / QB, 2), dim3(NT), smem, st, x, ldx, Q, D, H, cblob, NOC,
                     ce0, ce1, vblob, ve0, ve1, radius, tracks, logits, ldl, vis);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}
