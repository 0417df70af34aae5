// Chunk factors of the chunkwise gated delta rule: one workgroup per (chunk, b*h), all chunks in parallel.
//
// For the 64 tokens of a chunk (archbench/layers/nsgdn.py:240-249 algebra with beta folded into A's rows; the
// cumsum -> K K^T -> solve_tril steps of fla's GDN chunk forward, nsgdn.py:357-360):
//   G    chunk-local inclusive cumsum of g                                            -> Gc [BH][NT][64] fp32
//   A    beta_i (k_i . u_j) exp(G_i - G_j), strictly lower, on MFMA (fp32 in LDS)
//   Tm   (I + A)^-1: diagonal 16x16 blocks by Neumann products, blocks below by column chains (bf16x3 MFMA)
//                                                                                     -> Tm [BH][NT][packed]
//   P    s (q_i . u_j) exp(G_i - G_j) for i >= j                                      -> P  [BH][NT][packed]
// (packed: the ten 16 x 16 blocks on and below the diagonal, the rest being zero; gdn_chunk_common.h)
// u is the write key: u = k for the gated delta rule (SEPU false); with separate write keys (SEPU, the n-step
// family, archbench/layers/nsgdn.py:240-249 with L_ij = (k_i . u_j) gamma_i / gamma_j) u is loaded too and
// beta may be absent (row scale 1).
// The sweeps over the sequence (forward, recompute, reverse) read these instead of rebuilding them for every
// 64-wide V block, and the gradient kernel reads G.  Rows past the end of the sequence hold zero k, q
// and beta, which makes Tm the identity and P zero there.
#include <algorithm>

#include "gdn_chunk_common.h"
#include "gdn_launch.h"

namespace gdn {

// Persistent: workgroup x handles items x, x + gridDim.x, ... of the (b*h, chunk) grid (item = bh * NT + c), with
// the next item's k, q, g and beta prefetched into registers while the current one is factored, in two batches
// (k after the first barrier, q, g, beta after the second: 6% faster than all at once).
// LDS overlays keep a workgroup at about 50 KB (bf16, K = 128), so three share a CU: A (fp32) overlays Q row for
// row where the row pitches match (see factors_kq), and Tm overlays K once every wave has finished K U^T.
template <typename T, int K>
constexpr bool factors_a_on_q() { return (K + 16 / (int)sizeof(T)) * (int)sizeof(T) == (CH + 4) * 4; }

template <typename T, int K, bool SEPU>
__global__ __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 && !SEPU ? 3 : 2)))
void chunk_factors_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ u,
                          const float* __restrict__ g, const float* __restrict__ beta, T* __restrict__ gTm,
                          T* __restrict__ gP, float* __restrict__ gGc, int T_, int H, int NT, int nitems,
                          float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LF = CH + 4;
  constexpr bool A_ON_Q = factors_a_on_q<T, K>();
  static_assert(LC <= LK, "Tm must fit in the K tile");
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];  // K, then Tm (stride LC)
  __shared__ __attribute__((aligned(16))) T sQ[CH * LK];  // Q, then A where the pitches match
  __shared__ __attribute__((aligned(16))) T sU_[SEPU ? CH * LK : 8];
  T* sU = SEPU ? sU_ : sK;
  __shared__ __attribute__((aligned(16))) float sA_[A_ON_Q ? 4 : CH * LF];
  float* sA = A_ON_Q ? reinterpret_cast<float*>(sQ) : sA_;
  __shared__ __attribute__((aligned(16))) float sD[4 * DBLK];
  __shared__ __attribute__((aligned(16))) T sP[CH * LC];
  T* sTm = sK;
  __shared__ float sG[CH], sB[CH];

  const int w = wave_id(), l = lane_id();
  RegTile<T, CH, K, NTHR, true> rk, rq, ru;  // k, q, u are read once here: nontemporal
  RegTok rt;
  auto prefetch = [&](int it, int part) {
    const int bh = it / NT, c = it - bh * NT;
    const int b = bh / H, h = bh - b * H;
    const int nvalid = min(CH, T_ - c * CH);
    const int64_t row0 = ((int64_t)b * T_ + (int64_t)c * CH) * H + h;
    if (part != 2) {
      rk.load(k + row0 * K, (int64_t)H * K, nvalid);
      if constexpr (SEPU) ru.load(u + row0 * K, (int64_t)H * K, nvalid);
    }
    if (part != 1) {
      rq.load(q + row0 * K, (int64_t)H * K, nvalid);
      if (w == 0) rt.load(g, beta, row0, H, nvalid);
    }
  };
  if ((int)blockIdx.x < nitems) prefetch(blockIdx.x, 0);
  for (int it = blockIdx.x; it < nitems; it += gridDim.x) {
    rk.store(sK, LK);
    rq.store(sQ, LK);
    if constexpr (SEPU) ru.store(sU, LK);
    if (w == 0) {
      const float G = wave_inclusive_scan(rt.ok ? rt.g : 0.f);
      sG[l] = G;
      sB[l] = rt.ok ? rt.b : 0.f;
      gGc[(int64_t)it * CH + l] = G;
    }
    __syncthreads();
    const int itn = it + (int)gridDim.x;
    if (itn < nitems) prefetch(itn, 1);
    factors_kq<T, K, 1>(sK, sU, sQ, sG, sB, scale, sA, sP, w);
    __syncthreads();  // every wave done with K (Tm overwrites it); A written
    if (itn < nitems) prefetch(itn, 2);
    const f32x4 D = factors_diag<T>(sA, sD, sTm, w);
    __syncthreads();
    factors_merge<T>(D, sA, sD, sTm, w);
    __syncthreads();
    s2g_tri<T, NTHR, true>(gTm + (int64_t)it * CH_TRI_ELEMS, sTm, LC, threadIdx.x);
    s2g_tri<T, NTHR, true>(gP + (int64_t)it * CH_TRI_ELEMS, sP, LC, threadIdx.x);
    __syncthreads();  // LDS free for the next item
  }
}

template <typename T, int K, bool SEPU>
static hipError_t factors_k(const ChunkArgs& a) {
  const int nitems = a.NT * a.B * a.H;
  const int per_cu = sizeof(T) == 2 && !SEPU ? 3 : 2;  // workgroups resident per CU (LDS)
  dim3 grid(std::min(nitems, per_cu * device_cu_count()));
  chunk_factors_kernel<T, K, SEPU><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.u), a.g, a.beta,
      static_cast<T*>(a.ws.Tm), static_cast<T*>(a.ws.P), a.ws.Gc, a.T, a.H, a.NT, nitems, a.scale);
  return hipGetLastError();
}

template <bool SEPU>
static hipError_t factors_dispatch(const ChunkArgs& a) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return factors_k<bf16, 64, SEPU>(a);
    if (a.K == 128) return factors_k<bf16, 128, SEPU>(a);
  } else if constexpr (!SEPU) {  // separate write keys: bf16 only
    if (a.K == 64) return factors_k<float, 64, SEPU>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_factors(const ChunkArgs& a) {
  return a.u ? factors_dispatch<true>(a) : factors_dispatch<false>(a);
}

}  // namespace gdn
