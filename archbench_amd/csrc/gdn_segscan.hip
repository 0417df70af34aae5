// Scan across the segments of a segmented chunk sweep (sequence parallelism inside one GPU).
//
// A sequence of NS segments (the token-major tensors viewed as [B*NS, T/NS, H, .]) is swept in parallel: a
// prefix pass gives, per segment s and head, the state the segment leaves from a zero entering state (loc_s,
// [K][V]) and the segment's transition Phi_s ([K][K], so that leaving = Phi_s entering + loc_s).  This kernel
// then carries the state across the segments in order, one small product per segment:
//     forward:  S_0 = h0,     out_s = S_s,   S_{s+1} = Phi_s S_s + loc_s,           fin = S_NS   (= hT)
// and the state gradient backwards, with the transposed transitions:
//     reverse:  G_NS = dhT,   out_s = G_{s+1}, G_s = Phi_s^T G_{s+1} + dloc_s,     fin = G_0    (= dh0)
// (out_s: the state entering segment s, or the gradient w.r.t. the state leaving it).  All in fp32.
//
// One workgroup per (b*h, 64-column block of V), four waves: wave w carries rows w K/4 .. of the block, lane l
// its column.  Phi_s is staged in LDS as it is stored (row-major, coalesced reads, no bank conflicts); the product
// runs over k in blocks of four, so each 16-byte read of the staged Phi (the same address in every lane of the
// wave: a broadcast) serves four multiply-adds: forward, Phi[r][k..k+3] per row r; reverse, Phi[k+j][r..r+3]
// per j.  The carried block is staged as [k][c], one 4-byte read per lane per k.
#include <hip/hip_runtime.h>

#include "gdn_launch.h"

namespace gdn {

constexpr int SCAN_THREADS = 256;

template <int K, bool REVERSE>
__global__ __launch_bounds__(SCAN_THREADS) void seg_scan_kernel(const float* __restrict__ phi,
                                                               const float* __restrict__ loc,
                                                               const float* __restrict__ init,
                                                               float* __restrict__ outs, float* __restrict__ fin,
                                                               int NS, int H, int V) {
  constexpr int RW = K / 4;  // rows per wave
  __shared__ __attribute__((aligned(16))) float sM[K * K];   // Phi_s as stored: sM[r * K + k] = Phi(r, k)
  __shared__ __attribute__((aligned(16))) float sS[K * 64];  // carried block, [k][c]
  const int nvb = V / 64;
  const int bh = blockIdx.x / nvb, vb = blockIdx.x - bh * nvb;
  const int b = bh / H, h = bh - b * H;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int r0 = w * RW, c = vb * 64 + l;
  float acc[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) acc[i] = init ? init[((int64_t)bh * K + r0 + i) * V + c] : 0.f;
  for (int step = 0; step < NS; ++step) {
    const int s = REVERSE ? NS - 1 - step : step;
    const int64_t seg = (int64_t)(b * NS + s) * H + h;  // (b, s, h) in the segmented [B*NS, H, ...] layout
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      outs[(seg * K + r0 + i) * V + c] = acc[i];
      sS[(r0 + i) * 64 + l] = acc[i];
    }
    for (int idx = threadIdx.x; idx < K * K / 4; idx += SCAN_THREADS)
      reinterpret_cast<float4*>(sM)[idx] = reinterpret_cast<const float4*>(phi + seg * K * K)[idx];
    __syncthreads();
    float nxt[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) nxt[i] = loc[(seg * K + r0 + i) * V + c];
#pragma unroll 2
    for (int kb = 0; kb < K; kb += 4) {
      float sv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = sS[(kb + j) * 64 + l];
      if constexpr (!REVERSE) {
        // nxt[r] += sum_j Phi[r][kb + j] S[kb + j]
#pragma unroll
        for (int i = 0; i < RW; ++i) {
          const float4 m = *reinterpret_cast<const float4*>(sM + (r0 + i) * K + kb);
          nxt[i] += m.x * sv[0] + m.y * sv[1] + m.z * sv[2] + m.w * sv[3];
        }
      } else {
        // nxt[r] += sum_j Phi[kb + j][r] G[kb + j]
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i4 = 0; i4 < RW / 4; ++i4) {
            const float4 m = *reinterpret_cast<const float4*>(sM + (kb + j) * K + r0 + 4 * i4);
            nxt[4 * i4 + 0] += m.x * sv[j];
            nxt[4 * i4 + 1] += m.y * sv[j];
            nxt[4 * i4 + 2] += m.z * sv[j];
            nxt[4 * i4 + 3] += m.w * sv[j];
          }
      }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) acc[i] = nxt[i];
    __syncthreads();  // every wave is done with sS and sM before the next segment overwrites them
  }
  if (fin) {
#pragma unroll
    for (int i = 0; i < RW; ++i) fin[((int64_t)bh * K + r0 + i) * V + c] = acc[i];
  }
}

hipError_t launch_seg_scan(const float* phi, const float* loc, const float* init, float* outs, float* fin, int B,
                           int NS, int H, int K, int V, bool reverse, hipStream_t stream) {
  if (V % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((int64_t)B * H * (V / 64)));
  auto go = [&](auto kern) {
    kern<<<grid, SCAN_THREADS, 0, stream>>>(phi, loc, init, outs, fin, NS, H, V);
    return hipGetLastError();
  };
  if (K == 64) return reverse ? go(seg_scan_kernel<64, true>) : go(seg_scan_kernel<64, false>);
  if (K == 128) return reverse ? go(seg_scan_kernel<128, true>) : go(seg_scan_kernel<128, false>);
  return hipErrorInvalidValue;
}

}  // namespace gdn
