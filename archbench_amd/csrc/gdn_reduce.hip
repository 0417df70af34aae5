// Fixed-order column sums of per-workgroup partials: out[c] = sum over p of part[p * ld + c], the same order on
// every run (no atomics), so the parameter gradients built on it are deterministic.
#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int CS_COLS = 64;    // columns per workgroup (one per lane)
constexpr int CS_SLICES = 16;  // waves per workgroup, each summing every 16th partial

// One workgroup per 64 consecutive columns; wave s sums partials s, s + 16, ... in four interleaved chains
// (coalesced 256-byte rows), then the 16 wave sums are added in wave order.
__global__ __launch_bounds__(64 * CS_SLICES) void column_sum_kernel(const float* __restrict__ part, int64_t nparts,
                                                                    int64_t ld, int ncols, ColumnOut out) {
  __shared__ float red[CS_SLICES][CS_COLS];
  const int l = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int c = blockIdx.x * CS_COLS + l;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (c < ncols) {
    const float* src = part + c;
    int64_t p = sl;
    for (; p + 3 * CS_SLICES < nparts; p += 4 * CS_SLICES) {
      a0 += src[p * ld];
      a1 += src[(p + CS_SLICES) * ld];
      a2 += src[(p + 2 * CS_SLICES) * ld];
      a3 += src[(p + 3 * CS_SLICES) * ld];
    }
    for (; p < nparts; p += CS_SLICES) a0 += src[p * ld];
  }
  red[sl][l] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (sl == 0 && c < ncols) {
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < CS_SLICES; ++i) r += red[i][l];
    if (c < out.n[0]) {
      if (out.p[0]) out.p[0][c] = r;
    } else if (c < out.n[0] + out.n[1]) {
      if (out.p[1]) out.p[1][c - out.n[0]] = r;
    } else if (out.p[2]) {
      out.p[2][c - out.n[0] - out.n[1]] = r;
    }
  }
}

hipError_t launch_column_sum(const float* part, int64_t nparts, int64_t ld, ColumnOut out, hipStream_t stream) {
  const int ncols = out.n[0] + out.n[1] + out.n[2];
  if (ncols <= 0) return hipSuccess;
  column_sum_kernel<<<dim3((ncols + CS_COLS - 1) / CS_COLS), 64 * CS_SLICES, 0, stream>>>(part, nparts, ld, ncols,
                                                                                           out);
  return hipGetLastError();
}

}  // namespace gdn
