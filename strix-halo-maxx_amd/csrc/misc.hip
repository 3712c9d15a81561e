// Small device-side helpers for graph-replayed loops.
#include "common.h"

namespace {
__global__ void counter_add_kernel(int* p, int v) {
  if (threadIdx.x == 0) p[0] += v;
}

}  // namespace

// p[0] += v on the stream (a frame / step counter that a captured graph advances on every replay).
extern "C" int mx_counter_add(hipStream_t st, int* p, int v) {
  if (!p) return MX_ENULL;
  hipLaunchKernelGGL(counter_add_kernel, dim3(1), dim3(64), 0, st, p, v);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_ELAUNCH;
}

