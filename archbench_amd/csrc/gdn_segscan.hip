// Scan across the segments of a segmented chunk sweep (sequence parallelism inside one GPU).
//
// A sequence of NS segments (the token-major tensors viewed as [B*NS, T/NS, H, .]) is swept in parallel: a
// prefix pass gives, per segment s and head, the state the segment leaves from a zero entering state (loc_s,
// [K][V]; for the first segment from h0, so loc_0 = Phi_0 h0 + its local state) and the segment's transition
// Phi_s ([K][K], so that leaving = Phi_s entering + loc_s).  This kernel then carries the state across the
// segments in order, one small product per segment:
//     forward:  out_0 = S_0 = h0,  S_1 = loc_0,  S_{s+1} = Phi_s S_s + loc_s (s >= 1),  fin = S_NS   (= hT)
// and the state gradient backwards, with the transposed transitions (dloc_{NS-1} likewise already carrying dhT):
//     reverse:  out_{NS-1} = dhT,  G_{NS-1} = dloc_{NS-1},  G_s = Phi_s^T G_{s+1} + dloc_s,  out_s = G_{s+1},
//               fin = G_0 (= dh0)
// (out_s: the state entering segment s, or the gradient w.r.t. the state leaving it).  All in fp32.  Phi of the
// first (forward) or last (reverse) segment is never read, and without fin neither is the other end's: the main
// sweeps produce hT (from the last segment) and dh0 (from the first) themselves.
//
// One workgroup of 256 threads per (b*h, 16-column block of V): thread t carries column c = t & 15 of the block
// and RPL = K/16 rows of it, row(i) = i*16 + (t >> 4) forward and (t >> 4)*RPL + i in reverse.  Phi_s is staged
// row-major in LDS with a row pitch of K + 4 floats (coalesced 16-byte loads, prefetched into registers one segment
// ahead so the global latency overlaps the previous segment's product); the carried block is staged as [k][c].
//   forward  (out = Phi S):    lane reads Phi[row(i)][k .. k+3], one 16-byte read per row and block of four k;
//                              the four row groups of a wave are one row apart: distinct banks with this pitch.
//   reverse  (out = Phi^T G):  lane reads Phi[k][row(0) .. row(RPL-1)] (contiguous rows), RPL/4 16-byte reads per k;
//                              the row groups are RPL floats apart in one LDS row: distinct banks.
// The 16 lanes of a row group read the same LDS address (a broadcast).
#include <hip/hip_runtime.h>

#include "gdn_launch.h"

namespace gdn {

constexpr int SCAN_THREADS = 256;
constexpr int SCAN_COLS = 16;
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Loads segment `seg`'s Phi (16-byte pieces threadIdx.x + j * SCAN_THREADS) and the lane's rows of loc.
template <int K, int NPH, int RPL, bool REVERSE>
__device__ __forceinline__ void scan_fetch(const float* __restrict__ phi, const float* __restrict__ loc, int64_t seg,
                                           int rg, int c, int V, f32x4 (&pf)[NPH], float (&lf)[RPL]) {
  const f32x4* src = reinterpret_cast<const f32x4*>(phi + seg * K * K);
#pragma unroll
  for (int j = 0; j < NPH; ++j) pf[j] = src[threadIdx.x + j * SCAN_THREADS];
#pragma unroll
  for (int i = 0; i < RPL; ++i) lf[i] = loc[(seg * K + (REVERSE ? rg * RPL + i : i * 16 + rg)) * V + c];
}

template <int K, bool REVERSE>
__global__ __launch_bounds__(SCAN_THREADS) void seg_scan_kernel(const float* __restrict__ phi,
                                                               const float* __restrict__ loc,
                                                               const float* __restrict__ init,
                                                               float* __restrict__ outs, float* __restrict__ fin,
                                                               int NS, int H, int V) {
  constexpr int LDM = K + 4;                           // staged row pitch (floats)
  constexpr int RPL = K / 16;                          // rows per lane
  constexpr int NPH = K * K / 4 / SCAN_THREADS;        // 16-byte pieces of Phi per thread
  static_assert(NPH * 4 * SCAN_THREADS == K * K && RPL % 4 == 0, "scan tiling");
  __shared__ __attribute__((aligned(16))) float sM[K * LDM];         // Phi_s[r][k]
  __shared__ __attribute__((aligned(16))) float sS[K * SCAN_COLS];   // carried block, [k][c]
  const int ncb = V / SCAN_COLS;
  const int bh = blockIdx.x / ncb, cb = blockIdx.x - bh * ncb;
  const int b = bh / H, h = bh - b * H;
  const int cl = threadIdx.x & (SCAN_COLS - 1), rg = threadIdx.x >> 4;
  const int c = cb * SCAN_COLS + cl;
  auto row = [&](int i) { return REVERSE ? rg * RPL + i : i * 16 + rg; };
  // (b, s, h) in the segmented [B*NS, H, ...] layout
  auto seg_of = [&](int step) { return (int64_t)(b * NS + (REVERSE ? NS - 1 - step : step)) * H + h; };
  f32x4 pf[NPH];
  float lf[RPL], acc[RPL];
  scan_fetch<K, NPH, RPL, REVERSE>(phi, loc, seg_of(0), rg, c, V, pf, lf);
#pragma unroll
  for (int i = 0; i < RPL; ++i) acc[i] = init ? init[((int64_t)bh * K + row(i)) * V + c] : 0.f;
  for (int step = 0; step < NS; ++step) {
    const int64_t seg = seg_of(step);
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      outs[(seg * K + row(i)) * V + c] = acc[i];
      sS[row(i) * SCAN_COLS + cl] = acc[i];
    }
    if (step == NS - 1 && !fin) break;  // uniform: nothing reads the state past the last segment
    const bool prod = step > 0;         // the first local state already carries init
    if (prod) {
#pragma unroll
      for (int j = 0; j < NPH; ++j) {
        const int f = threadIdx.x + j * SCAN_THREADS;   // piece f of Phi: row f / (K/4), columns 4 (f % (K/4)) ..
        *reinterpret_cast<f32x4*>(sM + (f / (K / 4)) * LDM + (f % (K / 4)) * 4) = pf[j];
      }
    }
    float nxt[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) nxt[i] = lf[i];
    // the next segment's Phi and loc (the last step reloads its own)
    scan_fetch<K, NPH, RPL, REVERSE>(phi, loc, seg_of(step + 1 < NS ? step + 1 : step), rg, c, V, pf, lf);
    if (prod) __syncthreads();
#pragma unroll 2
    for (int kb = 0; kb < (prod ? K : 0); kb += 4) {
      float sv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = sS[(kb + j) * SCAN_COLS + cl];
      if constexpr (!REVERSE) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          const float4 m = *reinterpret_cast<const float4*>(sM + row(i) * LDM + kb);
          nxt[i] += m.x * sv[0] + m.y * sv[1] + m.z * sv[2] + m.w * sv[3];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int q = 0; q < RPL / 4; ++q) {
            const float4 m = *reinterpret_cast<const float4*>(sM + (kb + j) * LDM + rg * RPL + 4 * q);
            nxt[4 * q] += m.x * sv[j];
            nxt[4 * q + 1] += m.y * sv[j];
            nxt[4 * q + 2] += m.z * sv[j];
            nxt[4 * q + 3] += m.w * sv[j];
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RPL; ++i) acc[i] = nxt[i];
    __syncthreads();  // every wave is done with sS and sM before the next segment overwrites them
  }
  if (fin) {
#pragma unroll
    for (int i = 0; i < RPL; ++i) fin[((int64_t)bh * K + row(i)) * V + c] = acc[i];
  }
}

hipError_t launch_seg_scan(const float* phi, const float* loc, const float* init, float* outs, float* fin, int B,
                           int NS, int H, int K, int V, bool reverse, hipStream_t stream) {
  if (V % SCAN_COLS != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((int64_t)B * H * (V / SCAN_COLS)));
  auto go = [&](auto kern) {
    kern<<<grid, SCAN_THREADS, 0, stream>>>(phi, loc, init, outs, fin, NS, H, V);
    return hipGetLastError();
  };
  if (K == 64) return reverse ? go(seg_scan_kernel<64, true>) : go(seg_scan_kernel<64, false>);
  if (K == 128) return reverse ? go(seg_scan_kernel<128, true>) : go(seg_scan_kernel<128, false>);
  return hipErrorInvalidValue;
}

}  // namespace gdn
